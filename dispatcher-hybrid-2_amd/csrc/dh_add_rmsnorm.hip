// Residual add + RMSNorm of the parallel path (prefill / inference forward), for gfx950:
//   xo[r] = x[r] + y[r]                                   (rounded to the stream's dtype)
//   ho[r] = xo[r] * rsqrt(mean(xo[r]^2) + eps) * w        (fp32 math, rounded once)
// The residual stream of reference dispatcher_hybrid/modeling_dispatcher.py:210-212 / :225-227, :341-348
// (x = x + sublayer(norm1(x)); x + ffn(norm2(x))) adds a sublayer output and then normalises the
// sum for the next sublayer; this is that pair as one pass (two launches and a re-read of the sum
// otherwise). HBM-bound: 4 d s bytes per row (x, y read; xo, ho written; s = element size).
//
// One wave per row, four rows per 256-thread workgroup, no LDS and no barrier: each lane holds
// NCH 16-byte chunks of the row in registers (lane l owns elements (c*64 + l)*V .. +V-1), the sum
// of squares is reduced across the wave with xor shuffles, and the row is written from registers.
// EXACT (d == NCH*64*V) drops the per-chunk bounds test so every load issues before the first use.

#include "dh_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerWG = kThreads / 64;

template <typename T> struct Pack16;
template <> struct Pack16<bf16_t> {
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
template <> struct Pack16<float> {
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

template <typename T, int NCH, bool EXACT>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(const T* x, const T* y, const T* w, float eps,
                                                               T* xo, T* ho, int64_t rows, int d) {
  constexpr int V = 16 / sizeof(T);
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWG + (threadIdx.x >> 6);
  if (row >= rows) return;  // the whole wave leaves; the kernel has no barrier
  const int64_t base = row * (int64_t)d;
  // the norm weight is requested with the rows: xo may alias w for the compiler, so a load of w
  // after the xo stores would wait for them (two more round trips per row; 2.91 -> 2.75 us per
  // launch at 1024 x 1024 bf16 in captured graphs)
  uint4 xv[NCH], yv[NCH], wv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = (c * 64 + lane) * V;
    if (EXACT || e < d) {
      xv[c] = *reinterpret_cast<const uint4*>(x + base + e);
      yv[c] = *reinterpret_cast<const uint4*>(y + base + e);
      wv[c] = *reinterpret_cast<const uint4*>(w + e);
    } else {
      xv[c] = make_uint4(0, 0, 0, 0);
      yv[c] = xv[c];
      wv[c] = xv[c];
    }
  }
  float v[NCH][V];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float yf[V];
    Pack16<T>::unpack(xv[c], v[c]);
    Pack16<T>::unpack(yv[c], yf);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      v[c][j] = Elem<T>::round(v[c][j] + yf[j]);
      ss += v[c][j] * v[c][j];
    }
    const int e = (c * 64 + lane) * V;
    if (EXACT || e < d) *reinterpret_cast<uint4*>(xo + base + e) = Pack16<T>::pack(v[c]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float rstd = rsqrtf(ss / (float)d + eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = (c * 64 + lane) * V;
    if (EXACT || e < d) {
      float wf[V];
      Pack16<T>::unpack(wv[c], wf);
#pragma unroll
      for (int j = 0; j < V; ++j) wf[j] = (v[c][j] * rstd) * wf[j];
      *reinterpret_cast<uint4*>(ho + base + e) = Pack16<T>::pack(wf);
    }
  }
}

template <typename T, int NCH>
int launch_n(const void* x, const void* y, const void* w, float eps, void* xo, void* ho, int64_t rows, int d,
             hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const dim3 grid((unsigned)((rows + kRowsPerWG - 1) / kRowsPerWG));
  if (d == NCH * 64 * V)
    add_rmsnorm_kernel<T, NCH, true><<<grid, dim3(kThreads), 0, s>>>((const T*)x, (const T*)y, (const T*)w, eps,
                                                                     (T*)xo, (T*)ho, rows, d);
  else
    add_rmsnorm_kernel<T, NCH, false><<<grid, dim3(kThreads), 0, s>>>((const T*)x, (const T*)y, (const T*)w, eps,
                                                                      (T*)xo, (T*)ho, rows, d);
  return dh_check_launch("dh_add_rmsnorm");
}

template <typename T>
int launch(const void* x, const void* y, const void* w, float eps, void* xo, void* ho, int64_t rows, int d,
           hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const int nch = (d + 64 * V - 1) / (64 * V);
  if (nch <= 1) return launch_n<T, 1>(x, y, w, eps, xo, ho, rows, d, s);
  if (nch <= 2) return launch_n<T, 2>(x, y, w, eps, xo, ho, rows, d, s);
  if (nch <= 4) return launch_n<T, 4>(x, y, w, eps, xo, ho, rows, d, s);
  if (nch <= 8) return launch_n<T, 8>(x, y, w, eps, xo, ho, rows, d, s);
  return launch_n<T, 16>(x, y, w, eps, xo, ho, rows, d, s);
}

}  // namespace

extern "C" int dh_add_rmsnorm(int dtype, const void* x, const void* y, const void* weight, float eps, void* x_out,
                              void* h_out, int64_t rows, int d, void* stream) {
  const char* who = "dh_add_rmsnorm";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  const int V = dtype == DH_BF16 ? 8 : 4;
  DH_REQUIRE(rows >= 0 && rows <= ((int64_t)1 << 32), DH_ERR_INVALID_ARG, "%s: rows=%lld", who, (long long)rows);
  DH_REQUIRE(d >= V && d % V == 0 && d <= 16 * 64 * V, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: d=%d must be a multiple of %d in [%d, %d]", who, d, V, V, 16 * 64 * V);
  DH_REQUIRE(eps >= 0.f, DH_ERR_INVALID_ARG, "%s: eps=%g", who, (double)eps);
  if (rows == 0) return 0;
  DH_REQUIRE(x && y && weight && x_out && h_out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && (uintptr_t)weight % 16 == 0 &&
                 (uintptr_t)x_out % 16 == 0 && (uintptr_t)h_out % 16 == 0,
             DH_ERR_INVALID_ARG, "%s: operands need 16-byte alignment", who);
  hipStream_t s = (hipStream_t)stream;
  return dtype == DH_BF16 ? launch<bf16_t>(x, y, weight, eps, x_out, h_out, rows, d, s)
                          : launch<float>(x, y, weight, eps, x_out, h_out, rows, d, s);
}
