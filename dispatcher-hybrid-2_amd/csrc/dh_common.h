// Shared device and host helpers for libdh_mixer.so (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dh_mixer.h"

// ----------------------------------------------------------------------------------------------
// host side: thread-local error message + status helpers (defined in dh_abi.hip)
// ----------------------------------------------------------------------------------------------
int dh_fail(int status, const char* fmt, ...);
int dh_check_launch(const char* what);

#define DH_REQUIRE(cond, status, ...)            \
  do {                                           \
    if (!(cond)) return dh_fail((status), __VA_ARGS__); \
  } while (0)

// ----------------------------------------------------------------------------------------------
// element types: fp32 and bf16 (stored as raw uint16 bits)
// ----------------------------------------------------------------------------------------------
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t x) { return __uint_as_float(((uint32_t)x) << 16); }

// round-to-nearest-even fp32 -> bf16; NaN stays NaN. One v_cvt_pk_bf16_f32 (gfx950), issued by the
// compiler (which handles its hazards). Checked on the GPU against the integer form
// (u + 0x7fff + ((u >> 16) & 1)) >> 16 over all 2^32 inputs: equal for every non-NaN input (ties,
// subnormals, overflow to infinity), a NaN for every NaN.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// The dot product of two 16-byte chunks of 8 bf16 values on the dot-product unit: four
// v_dot2c_f32_bf16 steps, element pairs (0,1), (2,3), (4,5), (6,7) in that order, from 0. Every
// decode kernel whose result another path must equal bit for bit (the one-launch step and the
// graph of launches) forms its bf16 chunk products with this one function.
typedef __bf16 dh_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot8_bf16(const uint4& a, const uint4& b) {
  float s = 0.f;
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dh_bf16x2, a.x), __builtin_bit_cast(dh_bf16x2, b.x), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dh_bf16x2, a.y), __builtin_bit_cast(dh_bf16x2, b.y), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dh_bf16x2, a.z), __builtin_bit_cast(dh_bf16x2, b.z), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dh_bf16x2, a.w), __builtin_bit_cast(dh_bf16x2, b.w), s, false);
  return s;
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
  __device__ __forceinline__ static float round(float v) { return v; }
};
template <> struct Elem<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
  __device__ __forceinline__ static float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};

// Load 4 consecutive elements as fp32 (8-byte load for bf16, 16-byte for fp32). p must be aligned
// to 4 elements.
__device__ __forceinline__ void load4(const float* p, float (&o)[4]) {
  float4 v = *reinterpret_cast<const float4*>(p);
  o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
__device__ __forceinline__ void load4(const bf16_t* p, float (&o)[4]) {
  uint2 v = *reinterpret_cast<const uint2*>(p);
  o[0] = __uint_as_float(v.x << 16);
  o[1] = __uint_as_float(v.x & 0xffff0000u);
  o[2] = __uint_as_float(v.y << 16);
  o[3] = __uint_as_float(v.y & 0xffff0000u);
}

// logistic function from the hardware exp and reciprocal (v_exp_f32, v_rcp_f32: 1 ulp): 1 / (1 + e^-x).
// Saturates to exactly 1.0 for x >= ~17 (1 + e^-x rounds to 1, whose reciprocal is exact) and to
// exactly 0.0 for x <= -~89 (e^-x overflows to +inf).
__device__ __forceinline__ float dh_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// SiLU as torch evaluates it, x / (1 + e^-x) in fp32 with the library exp and an IEEE divide (the
// fp32 SwiGLU activation of the parallel path)
__device__ __forceinline__ float dh_silu_exact(float x) { return x / (1.0f + expf(-x)); }
// The same with the hardware exp (v_exp_f32, 12 instructions fewer), for bf16 inputs whose result is
// rounded to bf16: over every bf16 input the rounded result equals the rounded dh_silu_exact and
// torch's bf16 SiLU bit for bit (an exhaustive test covers all 65536 patterns). The IEEE divide
// stays: a reciprocal with one residual correction differs at x = -87.5 .. -88.5 and +inf.
__device__ __forceinline__ float dh_silu_bf16in(float x) { return x / (1.0f + __expf(-x)); }
// The same as dh_silu_bf16in with x times the reciprocal of 1 + e^-x refined by one Newton step in
// place of the IEEE divide (~6 instructions fewer): equal to it after rounding to bf16 for every
// bf16 input x >= -87 (exhaustive test; without the Newton step one input, 5.9375, rounds the other
// way). Below -87 the reciprocal leaves the normal range: callers take dh_silu_bf16in for any group
// of values holding such an input.
__device__ __forceinline__ float dh_silu_bf16in_rcp(float x) {
  const float d = 1.0f + __expf(-x);
  const float r = __builtin_amdgcn_rcpf(d);
  return x * __builtin_fmaf(r, __builtin_fmaf(-d, r, 1.0f), r);
}

// DPP lane move of a float: lanes in the rows of ROWMASK read the lane CTRL selects, others get 0
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}

// Full-wavefront (64 lanes) sum; every lane gets the result. DPP steps (no LDS traffic): butterflies
// within quads (quad_perm 1,0,3,2 and 2,3,0,1), then half-row and row mirrors complete each 16-lane
// row; row_bcast:15 and row_bcast:31 carry row sums upward so lane 63 holds the total, which
// readlane broadcasts.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xb1, 0xf>(v);    // quad_perm(1,0,3,2)
  v += dpp_move<0x4e, 0xf>(v);    // quad_perm(2,3,0,1)
  v += dpp_move<0x141, 0xf>(v);   // row_half_mirror
  v += dpp_move<0x140, 0xf>(v);   // row_mirror
  v += dpp_move<0x142, 0xa>(v);   // row_bcast:15 into rows 1, 3
  v += dpp_move<0x143, 0xc>(v);   // row_bcast:31 into rows 2, 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// A uniform value no thread of the launch writes (a decode position, a token row index), read
// through the constant address space: the compiler emits a scalar load, so waiting for it never
// waits for vector loads already in flight (those return in issue order), and it lands in an SGPR.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

// Scheduling fence: nothing moves across it. Placed after a burst of loads, every request of the
// burst is issued before the first wait for any of them (the scheduler otherwise interleaves
// arithmetic on early arrivals, with its waits, between the requests).
#define DH_ISSUE_FENCE() __builtin_amdgcn_sched_barrier(0)

__host__ __device__ __forceinline__ int64_t ring_offset(int j) { return ((int64_t)2 << j) - 2; }
__host__ __device__ __forceinline__ int64_t ring_mask(int j) { return ((int64_t)2 << j) - 1; }

// ----------------------------------------------------------------------------------------------
// argmax with torch.argmax's order: (value, index) a beats b when its value is larger, NaN above
// every number, the lower index on ties
// ----------------------------------------------------------------------------------------------
struct Cand {
  float v;
  int i;
};

__device__ __forceinline__ bool beats(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ void dpp_pair(float& v, int& i) {
  // lanes outside ROWMASK keep their own pair (old = own value), so the comparison is a no-op there
  const float ov = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
  const int oi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROWMASK, 0xf, false);
  if (beats(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}

// best (value, index) of a wave, in lane 63
__device__ __forceinline__ void wave_best(float& best, int& bidx) {
  dpp_pair<0xb1, 0xf>(best, bidx);      // quad_perm(1,0,3,2)
  dpp_pair<0x4e, 0xf>(best, bidx);      // quad_perm(2,3,0,1)
  dpp_pair<0x141, 0xf>(best, bidx);     // row_half_mirror
  dpp_pair<0x140, 0xf>(best, bidx);     // row_mirror
  dpp_pair<0x142, 0xa>(best, bidx);     // row_bcast:15 into rows 1, 3
  dpp_pair<0x143, 0xc>(best, bidx);     // row_bcast:31 into rows 2, 3
}
