// The parallel forward's tree mask with document resets, for gfx950:
//   mask[b, t, l] = [t >= 2^l] * [no EOT among ids[b, t - 2^l .. t - 1]]
// (reference dispatcher_hybrid/modeling_dispatcher.py:282-297, the level mask, and :311-323, the doc
// reset: doc(t) counts the EOTs strictly before t and level l's edge t <- t - 2^l is kept iff
// doc(t) = doc(t - 2^l), i.e. iff no EOT lies in [t - 2^l, t)). Values are exactly 0 or 1.
//
// One workgroup per row: each thread counts the EOTs of its contiguous chunk of positions, a block
// scan (wave prefix sums, then the wave totals in order) gives every position the count of EOTs
// before it, in LDS, and each thread writes the L values of its positions (a thread's rows are
// contiguous in the (b, T, L) output). One launch in place of the torch formula's eight (compare,
// casts, cumsum, subtract, gather, compare, product).
#include "dh_common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxT = 16384;                   // EOT counts of a row in LDS (64 KB)

template <typename T>
__global__ __launch_bounds__(kThreads) void tree_mask_kernel(const int64_t* ids, int64_t sid, int Tn, int L,
                                                             int64_t eot, T* out) {
  __shared__ int cnt[kMaxT];
  __shared__ int wsum[kThreads / 64];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ppt = (Tn + kThreads - 1) / kThreads;
  const int p0 = min(tid * ppt, Tn), p1 = min(p0 + ppt, Tn);
  const int64_t* row = ids + (int64_t)b * sid;
  int c = 0;
  for (int t = p0; t < p1; ++t) c += row[t] == eot ? 1 : 0;
  int incl = c;                                  // inclusive prefix over the wave's threads
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int run = incl - c;                            // EOTs before p0
  for (int w = 0; w < wave; ++w) run += wsum[w];
  for (int t = p0; t < p1; ++t) {
    cnt[t] = run;
    run += row[t] == eot ? 1 : 0;
  }
  __syncthreads();
  for (int t = p0; t < p1; ++t) {
    T* o = out + ((int64_t)b * Tn + t) * L;
    for (int l = 0; l < L; ++l) {
      const int lag = 1 << l;                    // L <= 30 (host check)
      const bool keep = t >= lag && cnt[t] == cnt[max(t - lag, 0)];
      Elem<T>::store(o + l, keep ? 1.f : 0.f);
    }
  }
}

}  // namespace

extern "C" int dh_tree_mask(int dtype, const int64_t* ids, int64_t ids_stride, int b, int T, int L, int64_t eot,
                            void* out, void* stream) {
  const char* who = "dh_tree_mask";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(b >= 1 && T >= 1 && L >= 1, DH_ERR_INVALID_ARG, "%s: b=%d T=%d L=%d must be >= 1", who, b, T, L);
  DH_REQUIRE(T <= kMaxT && L <= 30, DH_ERR_UNSUPPORTED_SHAPE, "%s: T=%d (<= %d) L=%d (<= 30)", who, T, kMaxT, L);
  DH_REQUIRE(ids && out && ids_stride >= T, DH_ERR_INVALID_ARG, "%s: null pointer or ids row stride < T", who);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_BF16)
    tree_mask_kernel<bf16_t><<<dim3(b), dim3(kThreads), 0, s>>>(ids, ids_stride, T, L, eot, (bf16_t*)out);
  else
    tree_mask_kernel<float><<<dim3(b), dim3(kThreads), 0, s>>>(ids, ids_stride, T, L, eot, (float*)out);
  return dh_check_launch(who);
}
