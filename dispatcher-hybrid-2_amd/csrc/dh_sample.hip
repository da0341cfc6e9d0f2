// Next-token selection on the device, for gfx950: greedy argmax over each row of logits.
//
// Semantics follow torch.argmax as fast_generate's greedy branch calls it (reference
// dispatcher_hybrid/modeling_dispatcher.py:426-441): the index of the largest value, the first
// such index on ties, and NaN counts as larger than every number (the first NaN wins).
//
// Work decomposition: two launches. The first splits every row into slices of kSlice elements, one
// workgroup (4 wave64s) per (slice, row): each thread requests all of its elements before
// comparing any, keeps its best (value, index), and DPP wave reductions plus one LDS step give the
// slice's candidate. The second launch reduces each row's candidates with the same ordering. A
// row of a 50k vocabulary thus streams through ~25 compute units instead of one.
#include <mutex>

#include "dh_common.h"

namespace {

constexpr int kSlice = 2048;              // elements per first-pass workgroup
constexpr int kT1 = 256;                  // first-pass threads: kSlice / kT1 = 8 elements each

template <typename T>
__global__ __launch_bounds__(kT1) void argmax_slices(const T* logits, int64_t row_stride, int V, Cand* cand) {
  __shared__ Cand wb[kT1 / 64];
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* row = logits + (int64_t)b * row_stride;
  constexpr int PT = kSlice / kT1;
  const int base = s * kSlice;
  float x[PT];
#pragma unroll
  for (int k = 0; k < PT; ++k) x[k] = Elem<T>::load(row + min(base + tid + k * kT1, V - 1));   // clamped
  float best = x[0];
  int bidx = min(base + tid, V - 1);
#pragma unroll
  for (int k = 1; k < PT; ++k) {
    const int i = base + tid + k * kT1;
    if (i < V && beats(x[k], i, best, bidx)) {
      best = x[k];
      bidx = i;
    }
  }
  wave_best(best, bidx);
  if (lane == 63) wb[wave] = Cand{best, bidx};
  __syncthreads();
  if (tid == 0) {
    Cand c = wb[0];
#pragma unroll
    for (int w = 1; w < kT1 / 64; ++w)
      if (beats(wb[w].v, wb[w].i, c.v, c.i)) c = wb[w];
    cand[(int64_t)b * gridDim.x + s] = c;
  }
}

__global__ __launch_bounds__(64) void argmax_final(const Cand* cand, int nslice, int64_t* out) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const Cand* cb = cand + (int64_t)b * nslice;
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  for (int j = lane; j < nslice; j += 64) {
    const Cand c = cb[j];
    if (beats(c.v, c.i, best, bidx)) {
      best = c.v;
      bidx = c.i;
    }
  }
  wave_best(best, bidx);
  if (lane == 63) out[b] = bidx;
}

// The greedy pick after a vocabulary head that wrote one candidate per workgroup (dh_decode_gemv
// with argmax_cand): one workgroup of 256 threads per row, every thread's candidates requested
// before any comparison (a loop of dependent loads would serialise them), wave reductions, one
// LDS step. Optionally the token is also stored at hist[b * hist_stride + *t_dev] (the position
// the decoder just advanced to), when that index is below hist_len.
constexpr int kRT = 256;
constexpr int kRPer = 32;                  // candidates per thread: up to 8192 per row

__global__ __launch_bounds__(kRT) void argmax_reduce_kernel(const Cand* cand, int ncand, int64_t* out,
                                                            const int64_t* t_dev, int64_t* hist,
                                                            int64_t hist_stride, int64_t hist_len) {
  __shared__ Cand wb[kRT / 64];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the history position first: a scalar load that then lands while the candidates are in flight
  const int64_t t = hist ? load_uniform(t_dev) : -1;
  const Cand* cb = cand + (int64_t)b * ncand;
  Cand c[kRPer];
#pragma unroll
  for (int k = 0; k < kRPer; ++k) {                   // only the row's candidates are requested
    c[k] = Cand{-INFINITY, 0x7fffffff};
    if (tid + k * kRT < ncand) c[k] = cb[tid + k * kRT];
  }
  float best = -INFINITY;
  int bidx = 0x7fffffff;
#pragma unroll
  for (int k = 0; k < kRPer; ++k)
    if (tid + k * kRT < ncand && beats(c[k].v, c[k].i, best, bidx)) {
      best = c[k].v;
      bidx = c[k].i;
    }
  wave_best(best, bidx);
  if (lane == 63) wb[wave] = Cand{best, bidx};
  __syncthreads();
  if (tid == 0) {
    Cand r = wb[0];
#pragma unroll
    for (int w = 1; w < kRT / 64; ++w)
      if (beats(wb[w].v, wb[w].i, r.v, r.i)) r = wb[w];
    out[b] = r.i;
    if (hist && t >= 0 && t < hist_len) hist[(int64_t)b * hist_stride + t] = r.i;
  }
}

// ---------------------------------------------------------------------------------------------
// Temperature / top-k sampling (reference modeling_dispatcher.py:426-441, the do_sample branch):
//   l   = float(logits[b]) / temperature
//   l_i = -inf where l_i < kth, kth = the top_k-th largest l (every element equal to kth stays)
//   out[b] ~ Categorical(softmax(l))
// One workgroup (16 wave64s) per row, the row held in registers (thread t owns elements
// [64t, 64t + 64), kept as order-preserving 32-bit keys; slots past V hold key 0, below every number).
// kth, exactly: tau = the top_k-th largest of the 1024 per-thread maxima is a lower bound (at least
// top_k elements are >= tau), so kth is the top_k-th largest of the elements >= tau; those are
// compacted into LDS (usually a few hundred) and radix-selected (four 8-bit histogram passes).
// When they exceed the LDS buffer (or top_k > 1024), a binary search over the key space with
// block-wide counts finds kth instead. Then weights exp(l_i - max) on the kept elements, a block
// prefix scan of the per-thread sums, and one uniform draw u in [0, 1) per row from Philox4x32-10
// (Salmon et al., SC'11) keyed by the seed with counter (offset, row): the token is the element
// whose cumulative weight interval, in index order, holds u * sum.
// ---------------------------------------------------------------------------------------------
constexpr int kST = 1024;                 // threads per row
constexpr int kSPT = 64;                  // elements per thread: V <= 65536
constexpr int kCap = 4096;                // candidate keys sorted in LDS

__device__ __forceinline__ uint32_t order_key(float f) {   // a < b  <=>  key(a) < key(b)
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Philox4x32-10: first output word for key `seed` and counter (ctr_lo, ctr_hi, c2, 0)
__device__ __forceinline__ uint32_t philox4x32_10(uint64_t seed, uint64_t ctr, uint32_t c2) {
  uint32_t x0 = (uint32_t)ctr, x1 = (uint32_t)(ctr >> 32), x2 = c2, x3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * x0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * x2;
    const uint32_t y0 = (uint32_t)(p1 >> 32) ^ x1 ^ k0;
    const uint32_t y2 = (uint32_t)(p0 >> 32) ^ x3 ^ k1;
    x1 = (uint32_t)p1;
    x3 = (uint32_t)p0;
    x0 = y0;
    x2 = y2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return x0;
}

// block-wide helpers over the kST threads; `red` holds kST / 64 entries; every thread gets the result
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kST / 64; ++w) m = fmaxf(m, red[w]);
  return m;
}
// exclusive prefix (in thread order) and total of a per-thread value
template <typename V>
__device__ __forceinline__ V block_scan(V v, V* red, V& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  V incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const V u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  __syncthreads();
  if (lane == 63) red[wave] = incl;
  __syncthreads();
  V base = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kST / 64; ++w) {
    base += w < wave ? red[w] : (V)0;
    total += red[w];
  }
  return base + incl - v;
}

// The k-th largest (duplicates counted) of the non-zero keys vals[0, n) in LDS, by radix select:
// four 8-bit passes from the top; each pass histograms the keys that share the digits found so far
// (LDS atomics), and one wave finds, from the top bin down, the bin where the running count reaches
// k. Returns 0 when fewer than k keys are non-zero. Callers synchronise before; every thread gets
// the result. hist: 256 entries; state: 4 (a pair per pass parity, so that thread 0 can reset the
// next pass's pair while other threads still read this one's).
// NP < 4 passes: keys whose low 32 - 8 NP bits are zero (the result keeps them zero).
template <int NP = 4>
__device__ __forceinline__ uint32_t radix_kth(const uint32_t* vals, int n, int k, uint32_t* hist, uint32_t* state) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0;
  uint32_t kk = (uint32_t)k;
  for (int pass = 0; pass < NP; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) hist[tid] = 0u;
    uint32_t* st = state + 2 * (pass & 1);
    if (tid == 0) {
      st[0] = 0xffffffffu;                           // not found
      st[1] = 0u;
    }
    __syncthreads();
    for (int i = tid; i < n; i += kST) {
      const uint32_t v = vals[i];
      if (v != 0u && ((uint64_t)v >> (shift + 8)) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {                                  // lane i: bins 255 - 4i .. 252 - 4i, descending
      uint32_t c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = hist[255 - 4 * lane - q];
      const uint32_t sum = c[0] + c[1] + c[2] + c[3];
      uint32_t incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = (uint32_t)__shfl_up((int)incl, o);
        if (lane >= o) incl += u;
      }
      const uint32_t excl = incl - sum;
      if (excl < kk && kk <= incl) {
        uint32_t acc = excl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (acc < kk && kk <= acc + c[q]) {
            st[0] = (uint32_t)(255 - 4 * lane - q);
            st[1] = kk - acc;
          }
          acc += c[q];
        }
      }
    }
    __syncthreads();
    const uint32_t d = st[0];
    if (d == 0xffffffffu) return 0u;                 // uniform: fewer than k keys
    kk = st[1];
    prefix = (prefix << 8) | d;
  }
  return prefix << (8 * (4 - NP));
}

// The ND dwords of bytes [mis + byte0, mis + byte0 + 4 ND) of a raw buffer whose base is 16-byte
// aligned (a row that starts mis < 16 bytes past an aligned address; mis is uniform): ND / 4 + 1
// aligned 16-byte loads, then a funnel shift by mis bytes -- the whole-dword part Q through a uniform
// branch (register indices stay static), the in-dword part, 8 (mis & 3) bits, by v_alignbit. Rows
// read with 16-byte loads at their own misaligned address cost ~45% more (measured on a
// 50257-element bf16 row, whose odd rows in a (B, V) tensor start 2 bytes off: 25-26 vs 17-18 us).
template <int ND, int Q>
__device__ __forceinline__ void shift_words(uint32_t (&w)[ND + 4], uint32_t sh) {
#pragma unroll
  for (int j = 0; j < ND; ++j) w[j] = __builtin_amdgcn_alignbit(w[j + Q + 1], w[j + Q], sh);
}
template <int ND>
__device__ __forceinline__ void row_words(__amdgpu_buffer_rsrc_t r, uint32_t byte0, uint32_t mis,
                                          uint32_t (&w)[ND + 4]) {
  const int nload = mis != 0u ? ND / 4 + 1 : ND / 4;  // uniform: an aligned row needs no extra load
#pragma unroll
  for (int c = 0; c <= ND / 4; ++c) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (c < nload)
      v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte0 + c * 16, 0, 0));
    w[4 * c] = v.x;
    w[4 * c + 1] = v.y;
    w[4 * c + 2] = v.z;
    w[4 * c + 3] = v.w;
  }
  if (mis == 0u) return;                               // uniform
  const uint32_t sh = (mis & 3u) * 8u;
  switch (mis >> 2) {                                  // uniform
    case 0: shift_words<ND, 0>(w, sh); break;
    case 1: shift_words<ND, 1>(w, sh); break;
    case 2: shift_words<ND, 2>(w, sh); break;
    default: shift_words<ND, 3>(w, sh); break;
  }
}
// a raw buffer over row[0, V) from the 16-byte aligned address at or below row; mis: row's offset
// from it. The range is checked per dword, so it is rounded up to whole dwords: for odd V in bf16
// the last element shares a dword with the 2 bytes after the row (never past a page: a dword
// holding an element is mapped whole); what those bytes hold is masked by the callers.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t aligned_row(const T* row, int V, uint32_t& mis) {
  mis = (uint32_t)(reinterpret_cast<uintptr_t>(row) & 15u);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(reinterpret_cast<const char*>(row) - mis), (short)0,
                                           (int)((mis + (uint32_t)V * sizeof(T) + 3u) & ~3u), 0x00020000);
}

template <typename T>
__global__ __launch_bounds__(kST) void sample_topk_kernel(const T* logits, int64_t row_stride, int V,
                                                          float temperature, int top_k, uint64_t seed,
                                                          const int64_t* offset_dev, int64_t* out, int64_t* tok_hist,
                                                          int64_t hist_stride, int64_t hist_len) {
  __shared__ uint32_t buf[kCap + 1];                   // + a slot for unselected writes
  __shared__ float fred[kST / 64];
  __shared__ uint32_t ured[kST / 64];
  __shared__ uint32_t hist[256], rstate[4];
  __shared__ int chosen, fallback;
  const int b = blockIdx.x, tid = threadIdx.x;
  const T* row = logits + (int64_t)b * row_stride;
  const int i0 = tid * kSPT;                           // this thread's elements: [i0, i0 + kSPT)
  const int nv = min(max(V - i0, 0), kSPT);
  const int64_t off = offset_dev ? load_uniform(offset_dev) : 0;

  // ---- the chunk as order keys of l = float(x) / temperature (key 0, below every number, past V).
  // Raw buffer loads: reads past the row return zero without touching memory; what lies past V
  // inside the last dword is masked by nv below.
  uint32_t mis;
  const __amdgpu_buffer_rsrc_t rsrc = aligned_row(row, V, mis);
  constexpr int ND = kSPT * (int)sizeof(T) / 4;        // dwords of the thread's elements
  uint32_t wd[ND + 4];
  row_words<ND>(rsrc, (uint32_t)(i0 * (int)sizeof(T)), mis, wd);
  uint32_t xk[kSPT];
#pragma unroll
  for (int j = 0; j < kSPT; ++j) {
    if constexpr (sizeof(T) == 2)
      xk[j] = (j & 1) ? (wd[j >> 1] & 0xffff0000u) : (wd[j >> 1] << 16);
    else
      xk[j] = wd[j];
  }
  uint32_t kmax = 0u;
#pragma unroll
  for (int j = 0; j < kSPT; ++j) {
    xk[j] = j < nv ? order_key(__uint_as_float(xk[j]) / temperature) : 0u;
    kmax = max(kmax, xk[j]);
  }
  if (tid == 0) {
    chosen = 0x7fffffff;
    fallback = -1;
  }
  uint32_t bm = kmax;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) bm = max(bm, (uint32_t)__shfl_xor((int)bm, o));
  if ((tid & 63) == 0) ured[tid >> 6] = bm;
  __syncthreads();
  uint32_t mkey = ured[0];
#pragma unroll
  for (int w = 1; w < kST / 64; ++w) mkey = max(mkey, ured[w]);
  const float M = key_value(mkey);

  // ---- kth largest (exact), as a key
  uint32_t kkey = 0u;                                  // 0: keep every element
  if (top_k > 0 && top_k < V) {                        // uniform
    bool found = false;
    if (top_k <= kST) {
      buf[tid] = kmax;
      __syncthreads();
      // tau: the top_k-th largest per-thread maximum (0 when fewer threads hold elements)
      const uint32_t tau = radix_kth(buf, kST, top_k, hist, rstate);
      uint32_t c = 0;
#pragma unroll
      for (int j = 0; j < kSPT; ++j) c += (xk[j] >= tau && xk[j] != 0u) ? 1u : 0u;
      uint32_t C;
      uint32_t r = block_scan(c, ured, C);
      if (C <= (uint32_t)kCap) {
#pragma unroll
        for (int j = 0; j < kSPT; ++j) {              // branch-free: unselected keys go to buf[kCap]
          const bool take = xk[j] >= tau && xk[j] != 0u;
          buf[take ? r : kCap] = xk[j];
          r += take ? 1u : 0u;
        }
        __syncthreads();
        kkey = radix_kth(buf, (int)C, top_k, hist, rstate);
        found = kkey != 0u;
      }
    }
    if (!found) {                                      // uniform: the largest v with count(key >= v) >= top_k
      uint32_t lo = 1u, hi = mkey;
      while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo + 1u) >> 1);
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < kSPT; ++j) c += xk[j] >= mid ? 1u : 0u;
        uint32_t cnt;
        (void)block_scan(c, ured, cnt);
        if (cnt >= (uint32_t)top_k) lo = mid; else hi = mid - 1u;
      }
      kkey = lo;
    }
  }
  // kept: l >= kth as floats (the reference's mask; -0.0 and +0.0 compare equal), weights in place
  const float kth = kkey ? key_value(kkey) : -INFINITY;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kSPT; ++j) {
    const float l = key_value(xk[j]);
    const float w = (xk[j] != 0u && l >= kth && l > -INFINITY) ? __expf(l - M) : 0.f;
    xk[j] = __float_as_uint(w);
    s += w;
  }
  float total;
  const float excl = block_scan(s, fred, total);

  // ---- the draw: the element whose cumulative interval (index order) holds u * total
  const uint32_t rnd = philox4x32_10(seed, (uint64_t)off, (uint32_t)b);
  const float target = (float)(rnd >> 8) * 0x1.0p-24f * total;
  if (s > 0.f) {
    int hit = 0x7fffffff, last = -1;
    float c = excl;
#pragma unroll
    for (int j = 0; j < kSPT; ++j) {
      const float w = __uint_as_float(xk[j]);
      const bool pos = w > 0.f;
      if (pos && hit == 0x7fffffff && target >= c && target < c + w) hit = i0 + j;
      last = pos ? i0 + j : last;
      c += w;
    }
    if (hit != 0x7fffffff) atomicMin(&chosen, hit);
    atomicMax(&fallback, last);
  }
  __syncthreads();
  if (tid == 0) {
    const int64_t tok = chosen != 0x7fffffff ? chosen : (fallback >= 0 ? fallback : 0);
    out[b] = tok;
    if (tok_hist && off >= 0 && off < hist_len) tok_hist[b * hist_stride + off] = tok;   // history at the position
  }
}

// bf16 logits with 0 < top_k <= kST: the same selection, weights and draw on 16-bit order keys of
// the logits themselves, two per register (the 32-bit keys of the kernel above take 64 registers per
// thread and spill). Division by a positive temperature is monotone and keeps distinct bf16 values
// distinct in fp32 (their spacing, 2^-8 relative, is far above fp32 rounding), so the order, the
// ties and the kept set of x and of l = x / temperature are the same. The candidates (keys >= tau)
// are compacted into LDS as (key << 16) | index, in index order, so after kth is known each thread
// walks only its own few entries: l = x / temperature and the weights exp(l - max l) are formed,
// as above, for the kept elements only, twice (for the sums, then for the draw), in the same order
// and association as the kernel above, whose output this kernel reproduces bit for bit (measured
// over 12,300 draws of tie-heavy, signed-zero, -inf and random rows). Rows whose candidates exceed
// the LDS list fall back to the key-space search and a walk over the registers.
__device__ __forceinline__ uint32_t key16x2(uint32_t w) {   // order keys of the two bf16 halves
  const uint32_t sgn = (w >> 15) & 0x00010001u;              // sign bit of each half
  return w ^ 0x80008000u ^ (sgn * 0x7fffu);                  // negative: ~h, else h | 0x8000
}
__device__ __forceinline__ float key16_value(uint32_t k) {  // inverse of one half's key
  const uint32_t h = (k & 0x8000u) ? (k ^ 0x8000u) : (k ^ 0xffffu);
  return __uint_as_float(h << 16);
}

__global__ __launch_bounds__(kST) void sample_topk_bf16_kernel(const bf16_t* logits, int64_t row_stride, int V,
                                                               float temperature, int top_k, uint64_t seed,
                                                               const int64_t* offset_dev, int64_t* out, int64_t* tok_hist,
                                                               int64_t hist_stride, int64_t hist_len) {
  constexpr int NP = kSPT / 2;                         // registers of packed key pairs
  __shared__ uint32_t buf[kCap + 1];
  __shared__ float fred[kST / 64];
  __shared__ uint32_t ured[kST / 64];
  __shared__ uint32_t hist[256], rstate[4];
  __shared__ int chosen, fallback;
  const int b = blockIdx.x, tid = threadIdx.x;
  const bf16_t* row = logits + (int64_t)b * row_stride;
  const int i0 = tid * kSPT;                           // this thread's elements: [i0, i0 + kSPT)
  const int nv = min(max(V - i0, 0), kSPT);
  const int64_t off = offset_dev ? load_uniform(offset_dev) : 0;

  // ---- keys: pair i holds elements 2i (low half) and 2i + 1 (high half); key 0 past V. The row
  // is read from the aligned address at or below it, as in sample_topk_kernel.
  uint32_t mis;
  const __amdgpu_buffer_rsrc_t rsrc = aligned_row(row, V, mis);
  uint32_t wd[NP + 4];
  row_words<NP>(rsrc, (uint32_t)(i0 * 2), mis, wd);
  uint32_t kp[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) kp[i] = key16x2(wd[i]);
  uint32_t kmax = 0u;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    kp[i] = 2 * i + 1 < nv ? kp[i] : (2 * i < nv ? (kp[i] & 0xffffu) : 0u);
    kmax = max(kmax, max(kp[i] & 0xffffu, kp[i] >> 16));
  }
  if (tid == 0) {
    chosen = 0x7fffffff;
    fallback = -1;
  }
  uint32_t bm = kmax;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) bm = max(bm, (uint32_t)__shfl_xor((int)bm, o));
  if ((tid & 63) == 0) ured[tid >> 6] = bm;
  __syncthreads();
  uint32_t mkey = ured[0];
#pragma unroll
  for (int w = 1; w < kST / 64; ++w) mkey = max(mkey, ured[w]);
  const float M = key16_value(mkey) / temperature;

  auto count_ge = [&](uint32_t thr) {                  // this thread's non-zero keys >= thr
    uint32_t c = 0;
    if (kmax < thr) return c;                          // most threads, once thr is near the top
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint32_t lo = kp[i] & 0xffffu, hi = kp[i] >> 16;
      c += (lo >= thr && lo != 0u) ? 1u : 0u;
      c += (hi >= thr && hi != 0u) ? 1u : 0u;
    }
    return c;
  };
  // ---- kth largest (exact), as a key: tau = the top_k-th largest per-thread maximum bounds it.
  // The keys >= tau (and -0.0 beside +0.0) are compacted into LDS in index order as (key << 16) |
  // index; kth is their top_k-th largest, and the kept elements are among them.
  buf[tid] = kmax << 16;
  __syncthreads();
  uint32_t tau = radix_kth<2>(buf, kST, top_k, hist, rstate) >> 16;
  tau = tau == 0x8000u ? 0x7fffu : tau;
  const uint32_t cnt = count_ge(tau);
  uint32_t C;
  const uint32_t r0 = block_scan(cnt, ured, C);
  uint32_t kkey = 0u;
  const bool compact = C <= (uint32_t)kCap;            // uniform
  if (compact) {
    if (cnt > 0u) {
      uint32_t r = r0;
#pragma unroll
      for (int i = 0; i < NP; ++i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t k = h ? kp[i] >> 16 : kp[i] & 0xffffu;
          if (k >= tau && k != 0u) buf[r++] = (k << 16) | (uint32_t)(i0 + 2 * i + h);
        }
      }
    }
    __syncthreads();
    kkey = radix_kth<2>(buf, (int)C, top_k, hist, rstate) >> 16;
  }
  if (kkey == 0u) {                                    // uniform: the largest v with count(key >= v) >= top_k
    uint32_t lo = 1u, hi = mkey;
    while (lo < hi) {
      const uint32_t mid = lo + ((hi - lo + 1u) >> 1);
      uint32_t n;
      (void)block_scan(count_ge(mid), ured, n);
      if (n >= (uint32_t)top_k) lo = mid; else hi = mid - 1u;
    }
    kkey = lo;
  }
  // kept: x >= kth as floats (-0.0 ties +0.0: key 0x7fff next to +0.0's 0x8000) and x > -inf
  // (key 0x007f); empty slots (key 0) are below both
  const uint32_t thr = max(kkey == 0x8000u ? 0x7fffu : kkey, 0x0080u);
  const bool listed = compact && thr >= tau;            // uniform: every kept element is in buf
  auto weight = [&](uint32_t k) { return __expf(key16_value(k) / temperature - M); };
  // this thread's kept elements in index order, from its compacted entries or its registers
  auto for_kept = [&](auto&& fn) {
    if (listed) {
      for (uint32_t e = r0; e < r0 + cnt; ++e) {
        const uint32_t v = buf[e];
        if ((v >> 16) >= thr) fn(v >> 16, (int)(v & 0xffffu));
      }
    } else if (kmax >= thr) {
#pragma unroll
      for (int i = 0; i < NP; ++i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t k = h ? kp[i] >> 16 : kp[i] & 0xffffu;
          if (k >= thr) fn(k, i0 + 2 * i + h);
        }
      }
    }
  };
  float s = 0.f;
  for_kept([&](uint32_t k, int) { s += weight(k); });
  float total;
  const float excl = block_scan(s, fred, total);

  // ---- the draw: the element whose cumulative interval (index order) holds u * total
  const uint32_t rnd = philox4x32_10(seed, (uint64_t)off, (uint32_t)b);
  const float target = (float)(rnd >> 8) * 0x1.0p-24f * total;
  if (s > 0.f) {
    int hit = 0x7fffffff, last = -1;
    float c = excl;
    for_kept([&](uint32_t k, int j) {
      const float w = weight(k);
      if (w > 0.f) {
        if (hit == 0x7fffffff && target >= c && target < c + w) hit = j;
        last = j;
      }
      c += w;
    });
    if (hit != 0x7fffffff) atomicMin(&chosen, hit);
    atomicMax(&fallback, last);
  }
  __syncthreads();
  if (tid == 0) {
    const int64_t tok = chosen != 0x7fffffff ? chosen : (fallback >= 0 ? fallback : 0);
    out[b] = tok;
    if (tok_hist && off >= 0 && off < hist_len) tok_hist[b * hist_stride + off] = tok;   // history at the position
  }
}

}  // namespace

extern "C" int dh_sample_topk_hist(int dtype, const void* logits, int64_t row_stride, int B, int V, float temperature,
                                   int top_k, uint64_t seed, const int64_t* offset_dev, int64_t* out, int64_t* tok_hist,
                                   int64_t hist_stride, int64_t hist_len, void* stream) {
  const char* who = tok_hist ? "dh_sample_topk_hist" : "dh_sample_topk";
  DH_REQUIRE(!tok_hist || (offset_dev && hist_stride >= hist_len && hist_len >= 0), DH_ERR_INVALID_ARG,
             "%s: a token history needs the position (offset_dev) and rows of hist_stride >= hist_len", who);
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && B <= 65535 && V >= 1 && row_stride >= V, DH_ERR_INVALID_ARG, "%s: B=%d V=%d row_stride=%lld",
             who, B, V, (long long)row_stride);
  DH_REQUIRE(V <= kST * kSPT, DH_ERR_UNSUPPORTED_SHAPE, "%s: V=%d exceeds %d", who, V, kST * kSPT);
  DH_REQUIRE(top_k >= 0 && top_k <= V, DH_ERR_INVALID_ARG, "%s: top_k=%d not in [0, V=%d] (0: no top-k)", who,
             top_k, V);
  DH_REQUIRE(temperature > 0.f && temperature < INFINITY, DH_ERR_INVALID_ARG, "%s: temperature %g must be positive",
             who, (double)temperature);
  DH_REQUIRE(logits && out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_BF16 && top_k > 0 && top_k <= kST && top_k < V)
    sample_topk_bf16_kernel<<<B, kST, 0, s>>>((const bf16_t*)logits, row_stride, V, temperature, top_k, seed,
                                               offset_dev, out, tok_hist, hist_stride, hist_len);
  else if (dtype == DH_BF16)
    sample_topk_kernel<bf16_t><<<B, kST, 0, s>>>((const bf16_t*)logits, row_stride, V, temperature, top_k, seed,
                                                  offset_dev, out, tok_hist, hist_stride, hist_len);
  else
    sample_topk_kernel<float><<<B, kST, 0, s>>>((const float*)logits, row_stride, V, temperature, top_k, seed,
                                                 offset_dev, out, tok_hist, hist_stride, hist_len);
  return dh_check_launch(who);
}

extern "C" int dh_sample_topk(int dtype, const void* logits, int64_t row_stride, int B, int V, float temperature,
                              int top_k, uint64_t seed, const int64_t* offset_dev, int64_t* out, void* stream) {
  return dh_sample_topk_hist(dtype, logits, row_stride, B, V, temperature, top_k, seed, offset_dev, out, nullptr, 0,
                             0, stream);
}

extern "C" int64_t dh_argmax_workspace_bytes(int B, int V) {
  return (int64_t)B * ((V + kSlice - 1) / kSlice) * (int64_t)sizeof(Cand);
}

extern "C" int dh_argmax(int dtype, const void* logits, int64_t row_stride, int B, int V, int64_t* out,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  const char* who = "dh_argmax";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && B <= 65535 && V >= 1 && row_stride >= V, DH_ERR_INVALID_ARG, "%s: B=%d V=%d row_stride=%lld",
             who, B, V, (long long)row_stride);
  DH_REQUIRE(logits && out && workspace, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(workspace_bytes >= dh_argmax_workspace_bytes(B, V), DH_ERR_INVALID_ARG,
             "%s: workspace of %lld bytes, needs %lld", who, (long long)workspace_bytes,
             (long long)dh_argmax_workspace_bytes(B, V));
  DH_REQUIRE((uintptr_t)workspace % 8 == 0, DH_ERR_INVALID_ARG, "%s: workspace needs 8-byte alignment", who);
  const int nslice = (V + kSlice - 1) / kSlice;
  Cand* cand = (Cand*)workspace;
  hipStream_t s = (hipStream_t)stream;
  dim3 g1(nslice, B);
  if (dtype == DH_BF16)
    argmax_slices<bf16_t><<<g1, kT1, 0, s>>>((const bf16_t*)logits, row_stride, V, cand);
  else
    argmax_slices<float><<<g1, kT1, 0, s>>>((const float*)logits, row_stride, V, cand);
  argmax_final<<<B, 64, 0, s>>>(cand, nslice, out);
  return dh_check_launch(who);
}

// ---------------------------------------------------------------------------------------------
// dh_argmax_noalloc: dh_argmax's two launches with the per-slice candidates in a fixed array of
// device memory that lives with the loaded code object (one copy per GPU, held until the process
// ends), for callers that cannot allocate. Nothing in it needs clearing: the final pass reads only
// the B * nslice candidates the first pass of the same call wrote. Calls that overlap on one GPU
// (two streams, two host threads) share the array and race.
// ---------------------------------------------------------------------------------------------
#define DH_ARGMAX_NOALLOC_CANDS 8192     /* B * ceil(V / 2048) candidates at most: 64 KiB */
static __device__ __align__(256) Cand scratch[DH_ARGMAX_NOALLOC_CANDS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
Cand* g_scratch_ptr[kMaxDevices] = {};

// The array's address on device `dev` (current): in host code `scratch` names a host-side stand-in,
// so kernels get the address hipGetSymbolAddress reports, looked up once per device.
int noalloc_scratch(int dev, Cand** out, const char* who) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return dh_fail(DH_ERR_LAUNCH_FAILED, "%s: hipGetSymbolAddress of the candidate scratch failed: %s", who,
                     hipGetErrorString(e));
    g_scratch_ptr[dev] = (Cand*)p;
  }
  *out = g_scratch_ptr[dev];
  return DH_OK;
}
}  // namespace

extern "C" int dh_argmax_noalloc(int dtype, const void* logits, int64_t row_stride, int B, int V, int64_t* out,
                                 void* stream) {
  const char* who = "dh_argmax_noalloc";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && B <= 65535 && V >= 1 && row_stride >= V, DH_ERR_INVALID_ARG, "%s: B=%d V=%d row_stride=%lld",
             who, B, V, (long long)row_stride);
  DH_REQUIRE(logits && out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  const int nslice = (V + kSlice - 1) / kSlice;
  DH_REQUIRE((int64_t)B * nslice <= DH_ARGMAX_NOALLOC_CANDS, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: B=%d rows of V=%d need %lld candidates, beyond the fixed scratch of %d (B * ceil(V / %d)); "
             "use dh_argmax with a workspace",
             who, B, V, (long long)B * nslice, DH_ARGMAX_NOALLOC_CANDS, kSlice);
  int dev = 0;
  DH_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, DH_ERR_LAUNCH_FAILED,
             "%s: no usable current device", who);
  Cand* cand = nullptr;
  const int st = noalloc_scratch(dev, &cand, who);
  if (st != DH_OK) return st;
  hipStream_t s = (hipStream_t)stream;
  dim3 g1(nslice, B);
  if (dtype == DH_BF16)
    argmax_slices<bf16_t><<<g1, kT1, 0, s>>>((const bf16_t*)logits, row_stride, V, cand);
  else
    argmax_slices<float><<<g1, kT1, 0, s>>>((const float*)logits, row_stride, V, cand);
  argmax_final<<<B, 64, 0, s>>>(cand, nslice, out);
  return dh_check_launch(who);
}

extern "C" int dh_argmax_reduce(const void* cand, int B, int ncand, int64_t* out, const int64_t* t_dev,
                                int64_t* hist, int64_t hist_stride, int64_t hist_len, void* stream) {
  const char* who = "dh_argmax_reduce";
  DH_REQUIRE(cand && out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(B >= 1 && ncand >= 1 && ncand <= kRT * kRPer, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: B=%d ncand=%d (1..%d candidates per row)", who, B, ncand, kRT * kRPer);
  DH_REQUIRE(!hist || (t_dev && hist_len >= 1 && hist_stride >= hist_len), DH_ERR_INVALID_ARG,
             "%s: a history needs t_dev and hist_stride >= hist_len >= 1", who);
  argmax_reduce_kernel<<<dim3(B), dim3(kRT), 0, (hipStream_t)stream>>>((const Cand*)cand, ncand, out, t_dev,
                                                                         hist, hist_stride, hist_len);
  return dh_check_launch(who);
}
