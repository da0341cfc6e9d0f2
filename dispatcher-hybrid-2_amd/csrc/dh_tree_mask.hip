// The parallel forward's tree mask with document resets, for gfx950:
//   mask[b, t, l] = [t >= 2^l] * [no EOT among ids[b, t - 2^l .. t - 1]]
// (reference dispatcher_hybrid/modeling_dispatcher.py:282-297, the level mask, and :311-323, the doc
// reset: doc(t) counts the EOTs strictly before t and level l's edge t <- t - 2^l is kept iff
// doc(t) = doc(t - 2^l), i.e. iff no EOT lies in [t - 2^l, t)). Values are exactly 0 or 1.
//
// With p(t) = the last EOT position before t (-1 if none), "no EOT in [t - 2^l, t)" is
// p(t) < t - 2^l, so each position needs p(t) alone. One 256-thread workgroup per (256-position
// slice, row), one position per thread: the workgroup takes the last EOT before its slice as a max
// over the row's earlier ids (strided, then wave and workgroup maxima), and the positions within
// the slice by an inclusive max-scan (wave shuffles, then the wave totals in order). Each thread
// writes its position's L values, packed two or four to a store when the row layout allows. One
// launch in place of the torch formula's eight (compare, casts, cumsum, subtract, gather, compare,
// product).
#include "dh_common.h"

namespace {

constexpr int kTPB = 256;

__device__ __forceinline__ int wave_max_int(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

template <typename T>
__device__ __forceinline__ uint32_t mask_bits(bool v) {
  // the bit pattern of 1.0 or 0.0 in T
  if constexpr (sizeof(T) == 2) return v ? 0x3f80u : 0u;
  else return v ? 0x3f800000u : 0u;
}

template <typename T>
__global__ __launch_bounds__(kTPB) void tree_mask_kernel(const int64_t* ids, int64_t sid, int Tn, int L, int64_t eot,
                                                         T* out) {
  __shared__ int wred[kTPB / 64];
  const int b = blockIdx.y, t0 = blockIdx.x * kTPB, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t* row = ids + (int64_t)b * sid;
  // the last EOT before the slice
  int before = -1;
  for (int s = tid; s < t0; s += kTPB)
    if (row[s] == eot) before = s;                      // s grows: the last hit is the max
  before = wave_max_int(before);
  if (lane == 0) wred[wave] = before;
  __syncthreads();
  before = max(max(wred[0], wred[1]), max(wred[2], wred[3]));
  __syncthreads();                                      // wred is reused below
  // inclusive max-scan of (EOT at s ? s : -1) over the slice, then p(t) = the value at t - 1
  const int t = t0 + tid;
  int v = (t < Tn && row[t] == eot) ? t : -1;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o);
    if (lane >= o) v = max(v, u);
  }
  if (lane == 63) wred[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v = max(v, wred[w]);
  int p = __shfl_up(v, 1);                              // inclusive scan at t - 1 ...
  if (lane == 0) p = wave > 0 ? wred[wave - 1] : -1;   // ... or the earlier waves' maximum
  for (int w = 0; w < wave - 1; ++w) p = max(p, wred[w]);
  p = max(p, before);
  if (t >= Tn) return;
  T* o = out + ((int64_t)b * Tn + t) * L;
  auto bit = [&](int l) {
    const int lag = 1 << l;                              // L <= 30 (host check)
    return t >= lag && p < t - lag;
  };
  if ((L & 3) == 0) {                                    // 4 values per 8-byte store (rows 8-byte aligned)
    for (int l = 0; l < L; l += 4) {
      if constexpr (sizeof(T) == 2) {
        const uint32_t lo = mask_bits<T>(bit(l)) | (mask_bits<T>(bit(l + 1)) << 16);
        const uint32_t hi = mask_bits<T>(bit(l + 2)) | (mask_bits<T>(bit(l + 3)) << 16);
        *reinterpret_cast<uint2*>(o + l) = make_uint2(lo, hi);
      } else {
        *reinterpret_cast<uint4*>(o + l) = make_uint4(mask_bits<T>(bit(l)), mask_bits<T>(bit(l + 1)),
                                                      mask_bits<T>(bit(l + 2)), mask_bits<T>(bit(l + 3)));
      }
    }
  } else {
    for (int l = 0; l < L; ++l) Elem<T>::store(o + l, bit(l) ? 1.f : 0.f);
  }
}

}  // namespace

extern "C" int dh_tree_mask(int dtype, const int64_t* ids, int64_t ids_stride, int b, int T, int L, int64_t eot,
                            void* out, void* stream) {
  const char* who = "dh_tree_mask";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(b >= 1 && T >= 1 && L >= 1, DH_ERR_INVALID_ARG, "%s: b=%d T=%d L=%d must be >= 1", who, b, T, L);
  DH_REQUIRE(T <= 16384 && L <= 30 && b <= 65535, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: T=%d (<= 16384) L=%d (<= 30) b=%d (<= 65535)", who, T, L, b);
  DH_REQUIRE(ids && out && ids_stride >= T, DH_ERR_INVALID_ARG, "%s: null pointer or ids row stride < T", who);
  DH_REQUIRE((uintptr_t)out % 16 == 0, DH_ERR_INVALID_ARG, "%s: out needs 16-byte alignment", who);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((T + kTPB - 1) / kTPB, b);
  if (dtype == DH_BF16)
    tree_mask_kernel<bf16_t><<<grid, dim3(kTPB), 0, s>>>(ids, ids_stride, T, L, eot, (bf16_t*)out);
  else
    tree_mask_kernel<float><<<grid, dim3(kTPB), 0, s>>>(ids, ids_stride, T, L, eot, (float*)out);
  return dh_check_launch(who);
}
