// Next-token selection on the device, for gfx950: greedy argmax over each row of logits.
//
// Semantics follow torch.argmax as fast_generate's greedy branch calls it (reference
// dispatcher_hybrid/modeling_dispatcher.py:426-441): the index of the largest value, the first
// such index on ties, and NaN counts as larger than every number (the first NaN wins).
//
// Work decomposition: one workgroup (16 wave64s) per row. Every thread requests all of its
// elements (index tid + 1024*k) before comparing any, keeps its best (value, index), then DPP wave
// reductions and one LDS step across the waves pick the row's winner.
#include "dh_common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxPerThread = 64;        // V <= 65536

// a beats b: larger value, NaN above all numbers, lower index on ties
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

template <typename T, int PT>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const T* logits, int64_t row_stride, int V, int64_t* out) {
  __shared__ float bv[kWaves];
  __shared__ int bi[kWaves];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* row = logits + (int64_t)b * row_stride;
  float x[PT];
#pragma unroll
  for (int k = 0; k < PT; ++k) x[k] = Elem<T>::load(row + min(tid + k * kThreads, V - 1));   // clamped
  float best = x[0];
  int bidx = tid < V ? tid : V - 1;
#pragma unroll
  for (int k = 1; k < PT; ++k) {
    const int i = tid + k * kThreads;
    if (i < V && beats(x[k], i, best, bidx)) {
      best = x[k];
      bidx = i;
    }
  }
  dpp_pair<0xb1, 0xf>(best, bidx);      // quad_perm(1,0,3,2)
  dpp_pair<0x4e, 0xf>(best, bidx);      // quad_perm(2,3,0,1)
  dpp_pair<0x141, 0xf>(best, bidx);     // row_half_mirror
  dpp_pair<0x140, 0xf>(best, bidx);     // row_mirror
  dpp_pair<0x142, 0xa>(best, bidx);     // row_bcast:15 into rows 1, 3
  dpp_pair<0x143, 0xc>(best, bidx);     // row_bcast:31 into rows 2, 3
  if (lane == 63) {
    bv[wave] = best;
    bi[wave] = bidx;
  }
  __syncthreads();
  if (tid == 0) {
    float v = bv[0];
    int i = bi[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      if (beats(bv[w], bi[w], v, i)) {
        v = bv[w];
        i = bi[w];
      }
    out[b] = i;
  }
}

template <typename T>
void launch_argmax(const T* logits, int64_t row_stride, int B, int V, int64_t* out, hipStream_t s) {
  const int pt = (V + kThreads - 1) / kThreads;
  if (pt <= 8) argmax_kernel<T, 8><<<B, kThreads, 0, s>>>(logits, row_stride, V, out);
  else if (pt <= 16) argmax_kernel<T, 16><<<B, kThreads, 0, s>>>(logits, row_stride, V, out);
  else if (pt <= 32) argmax_kernel<T, 32><<<B, kThreads, 0, s>>>(logits, row_stride, V, out);
  else argmax_kernel<T, kMaxPerThread><<<B, kThreads, 0, s>>>(logits, row_stride, V, out);
}

}  // namespace

extern "C" int dh_argmax(int dtype, const void* logits, int64_t row_stride, int B, int V, int64_t* out,
                         void* stream) {
  const char* who = "dh_argmax";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && V >= 1 && row_stride >= V, DH_ERR_INVALID_ARG, "%s: B=%d V=%d row_stride=%lld", who, B, V,
             (long long)row_stride);
  DH_REQUIRE(V <= kThreads * kMaxPerThread, DH_ERR_UNSUPPORTED_SHAPE, "%s: V=%d exceeds %d", who, V,
             kThreads * kMaxPerThread);
  DH_REQUIRE(logits && out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_BF16)
    launch_argmax<bf16_t>((const bf16_t*)logits, row_stride, B, V, out, s);
  else
    launch_argmax<float>((const float*)logits, row_stride, B, V, out, s);
  return dh_check_launch(who);
}
