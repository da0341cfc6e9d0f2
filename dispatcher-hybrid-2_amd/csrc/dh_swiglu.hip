// SwiGLU activation of the parallel path (prefill / training-free forward), for gfx950:
//   out = silu(gate) * up,   silu(x) = x / (1 + e^-x)
// at the eager bf16 rounding points of reference dispatcher_hybrid/modeling_dispatcher.py
// (SwiGLU.forward: F.silu(linear_gate(h)) * linear_up(h)): silu evaluated in fp32 and rounded to
// bf16, the product formed in fp32 and rounded again. fp32 tensors: no rounding.
//
// One pass over the two (n) operands instead of two launches (silu, then the product) and a
// rounded intermediate in HBM. HBM-bound: 3 n s bytes (s = element size). Each thread moves 16-byte
// vectors (8 bf16 / 4 fp32) in a grid-stride loop; a scalar tail covers n % 8.

#include "dh_common.h"

namespace {

constexpr int kThreads = 256;

// 16 bytes of elements as fp32 and back
template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = __uint_as_float(w[j] << 16);
      o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static uint4 pack(const float (&o)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (uint32_t)f32_to_bf16(o[2 * j]) | ((uint32_t)f32_to_bf16(o[2 * j + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const uint4& v, float (&o)[4]) {
    o[0] = __uint_as_float(v.x);
    o[1] = __uint_as_float(v.y);
    o[2] = __uint_as_float(v.z);
    o[3] = __uint_as_float(v.w);
  }
  __device__ __forceinline__ static uint4 pack(const float (&o)[4]) {
    return make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3]));
  }
};

// bf16 inputs: the hardware-exp form (equal after rounding for every bf16 input); fp32: torch's
template <typename T>
__device__ __forceinline__ float silu_of(float x) {
  if constexpr (sizeof(T) == 2) return dh_silu_bf16in(x);
  else return dh_silu_exact(x);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const T* g, const T* u,
                                                            T* out, int64_t n) {
  constexpr int V = 16 / sizeof(T);
  const int64_t nvec = n / V;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nvec; i += stride) {
    const uint4 gv = reinterpret_cast<const uint4*>(g)[i];
    const uint4 uv = reinterpret_cast<const uint4*>(u)[i];
    float gf[V], uf[V];
    Vec16<T>::unpack(gv, gf);
    Vec16<T>::unpack(uv, uf);
#pragma unroll
    for (int e = 0; e < V; ++e) gf[e] = Elem<T>::round(Elem<T>::round(silu_of<T>(gf[e])) * uf[e]);
    reinterpret_cast<uint4*>(out)[i] = Vec16<T>::pack(gf);
  }
  // tail (n % V elements): the first threads of the grid
  const int64_t t = nvec * V + (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t < n) {
    const float s = Elem<T>::round(silu_of<T>(Elem<T>::load(g + t)));
    Elem<T>::store(out + t, Elem<T>::round(s * Elem<T>::load(u + t)));
  }
}

template <typename T>
int launch(const void* g, const void* u, void* out, int64_t n, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const int64_t nvec = n / V;
  int64_t blocks = (nvec + kThreads - 1) / kThreads;
  blocks = blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks);   // grid-stride past 8192 x 256 vectors
  silu_mul_kernel<T><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>((const T*)g, (const T*)u, (T*)out, n);
  return dh_check_launch("dh_silu_mul");
}

}  // namespace

extern "C" int dh_silu_mul(int dtype, const void* gate, const void* up, void* out, int64_t n, void* stream) {
  const char* who = "dh_silu_mul";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(n >= 0, DH_ERR_INVALID_ARG, "%s: n=%lld", who, (long long)n);
  if (n == 0) return 0;
  DH_REQUIRE(gate && up && out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE((uintptr_t)gate % 16 == 0 && (uintptr_t)up % 16 == 0 && (uintptr_t)out % 16 == 0,
             DH_ERR_INVALID_ARG, "%s: operands need 16-byte alignment", who);
  hipStream_t s = (hipStream_t)stream;
  return dtype == DH_BF16 ? launch<bf16_t>(gate, up, out, n, s) : launch<float>(gate, up, out, n, s);
}
