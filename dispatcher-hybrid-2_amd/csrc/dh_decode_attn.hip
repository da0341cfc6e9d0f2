// One decode step of a windowed RoPE attention layer, for gfx950: the rotation of the new query and
// key, the key/value cache write at the device position t, the scores over the window, the softmax
// and the value average, in one launch.
//
// Semantics (reference dispatcher_hybrid/decoding.py:411-435 graph step and :247-266 eager step;
// modeling_dispatcher.py:163-166 rope):
//   (q', k')   = rope(q[b,h], t), rope(k[b,h], t)     interleaved pairs: (x0 c - x1 s, x0 s + x1 c)
//   K[b,h,t]   = k' ; V[b,h,t] = v[b,h]
//   s_j        = (q' . K[b,h,j]) / sqrt(hd)            j in [lo, t], lo = max(0, t+1-window) (window > 0)
//   p          = softmax_j(s)                          (fp32 softmax, as the eager step computes it)
//   y[b,h]     = sum_j p_j V[b,h,j]
// bf16 mode rounds where the eager bf16 step rounds: each rope product and sum, the q'.K matmul
// output, its division by sqrt(hd), the softmax output and the value average.
//
// Work decomposition: one workgroup (8 wave64s) per (head, batch row). Pass 1 gives every thread
// one window position per sweep and the thread computes that position's full dot product from its
// key row (hd elements, contiguous in the head-major cache); the scores stay in LDS. A block
// reduction gives the maximum and the sum of exponentials. Pass 2 splits the window over the 8
// waves; a wave's 16-byte loads cover whole value rows (lane -> row slot, chunk of the row) and
// accumulate p_j V[j] in fp32, then the row slots and the waves are summed. The key rows of the
// first two sweeps and the first block of value rows are requested as soon as t is known, so the
// launch waits for memory about twice. The new position t is taken from LDS (the rotated key and
// the value computed in this launch), never read back from the cache the same launch writes.
#include "dh_common.h"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxHd = 128;
constexpr int kMaxWindow = 16384;   // scores held in LDS (64 KB)

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  int64_t qkv_bstride;
  const void* cos;
  const void* sin;
  void* K;
  void* V;
  const int64_t* t_dev;
  void* y;
  int64_t y_bstride;
  int H, Tmax, window;
  float scale;            // sqrt(hd): scores are divided by it
};

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xb1, 0xf>(v));
  v = fmaxf(v, dpp_move<0x4e, 0xf>(v));
  v = fmaxf(v, dpp_move<0x141, 0xf>(v));
  v = fmaxf(v, dpp_move<0x140, 0xf>(v));
  // row broadcasts fill the other rows' lanes with 0 (bound_ctrl): take max with the lane itself
  // only where the source row exists, which the row masks select
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// an element's raw bits (bf16 zero-extended), converted to fp32 separately
__device__ __forceinline__ uint32_t raw_load(const bf16_t* p) { return *p; }
__device__ __forceinline__ uint32_t raw_load(const float* p) { return __float_as_uint(*p); }
template <typename T> __device__ __forceinline__ float raw_f(uint32_t r);
template <> __device__ __forceinline__ float raw_f<bf16_t>(uint32_t r) { return __uint_as_float(r << 16); }
template <> __device__ __forceinline__ float raw_f<float>(uint32_t r) { return __uint_as_float(r); }

template <typename T, int HD>
__global__ __launch_bounds__(kThreads) void decode_attention_kernel(AttnArgs a) {
  extern __shared__ float sc[];                       // scores / probabilities of the window
  __shared__ float qs[kMaxHd], ks[kMaxHd], vs[kMaxHd];
  __shared__ float red[kWaves];
  __shared__ float part[kWaves][kMaxHd];
  constexpr int VE = 16 / (int)sizeof(T);             // elements per 16-byte chunk
  constexpr int LPR = HD / VE;                        // lanes per cache row in pass 2
  constexpr int RPI = 64 / LPR;                       // rows per wave load instruction
  constexpr int KCH = HD / VE;                        // 16-byte chunks per cache row
  constexpr int KP = KCH <= 8 ? 2 : 1;                // pass-1 sweeps whose key rows are prefetched
  constexpr int CH = KCH <= 8 ? 16 : 8;               // pass-2 loads in flight per lane
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t = load_uniform(a.t_dev);
  if (t < 0 || t >= a.Tmax) return;                   // workgroup-uniform: nothing to do
  const int lo = a.window > 0 ? (int)max((int64_t)0, t + 1 - a.window) : 0;
  const int n = (int)t - lo + 1;
  const int nc = n - 1;                               // cached positions; index n-1 is t itself
  const int64_t head_off = ((int64_t)b * a.H + h) * a.Tmax * HD;  // (b, h) rows of the caches
  T* Kh = (T*)a.K + head_off;
  T* Vh = (T*)a.V + head_off;

  // ---- the rotation's operands first (q, k, v pairs of this thread and the angle at t): loads
  // return in issue order, so the rotation and the cache write below wait only for these while the
  // key and value requests behind them are in flight
  // (raw bits, loaded by every thread at a clamped index: a branch or a conversion here would put
  // a wait for them ahead of the key and value requests)
  const bool roper = tid < HD / 2;
  uint32_t rop[8];
  {
    const int pt = min(tid, HD / 2 - 1);
    const int64_t base = (int64_t)b * a.qkv_bstride + (int64_t)h * HD + 2 * pt;
    rop[0] = raw_load((const T*)a.cos + t * (HD / 2) + pt);
    rop[1] = raw_load((const T*)a.sin + t * (HD / 2) + pt);
    rop[2] = raw_load((const T*)a.q + base);
    rop[3] = raw_load((const T*)a.q + base + 1);
    rop[4] = raw_load((const T*)a.k + base);
    rop[5] = raw_load((const T*)a.k + base + 1);
    rop[6] = raw_load((const T*)a.v + base);
    rop[7] = raw_load((const T*)a.v + base + 1);
  }
  DH_ISSUE_FENCE();

  // ---- requests that need only t: this thread's first key row (pass 1) and its first block of
  // value chunks (pass 2); they fly while the new key is rotated. Rows are clamped into the cached
  // range, so every load reads a written cache row (results past the range are discarded).
  const int ck = nc > 0 ? nc - 1 : 0;
  uint4 krow[KP][KCH];
#pragma unroll
  for (int q = 0; q < KP; ++q) {
    const int j = lo + min(tid + q * kThreads, ck);
#pragma unroll
    for (int c = 0; c < KCH; ++c) krow[q][c] = reinterpret_cast<const uint4*>(Kh + (int64_t)j * HD)[c];
  }
  const int per = (nc + kWaves - 1) / kWaves;
  const int j0 = wave * per, j1 = min(nc, j0 + per);
  const int slot = lane / LPR, dg = lane % LPR;       // row within an instruction, 16-byte chunk of the row
  uint4 vrow[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int i = min(j0 + u * RPI + slot, ck);
    vrow[u] = reinterpret_cast<const uint4*>(Vh + (int64_t)(lo + i) * HD)[dg];
  }
  DH_ISSUE_FENCE();

  // ---- rope of q and k at position t, cache write of (k', v) at t
  if (roper) {
    asm volatile("" : "+v"(rop[0]), "+v"(rop[1]), "+v"(rop[2]), "+v"(rop[3]), "+v"(rop[4]), "+v"(rop[5]),
                 "+v"(rop[6]), "+v"(rop[7]));           // converted here, after the key/value requests
    const float c = raw_f<T>(rop[0]), s = raw_f<T>(rop[1]);
    const float q0 = raw_f<T>(rop[2]), q1 = raw_f<T>(rop[3]);
    const float k0 = raw_f<T>(rop[4]), k1 = raw_f<T>(rop[5]);
    const float v0 = raw_f<T>(rop[6]), v1 = raw_f<T>(rop[7]);
    typedef Elem<T> E;
    float qr0, qr1, kr0, kr1;
    {
      // every product rounded on its own (torch evaluates them as separate tensor ops): no FMA
#pragma clang fp contract(off)
      qr0 = E::round(E::round(q0 * c) - E::round(q1 * s));
      qr1 = E::round(E::round(q0 * s) + E::round(q1 * c));
      kr0 = E::round(E::round(k0 * c) - E::round(k1 * s));
      kr1 = E::round(E::round(k0 * s) + E::round(k1 * c));
    }
    qs[2 * tid] = qr0; qs[2 * tid + 1] = qr1;
    ks[2 * tid] = kr0; ks[2 * tid + 1] = kr1;
    vs[2 * tid] = v0; vs[2 * tid + 1] = v1;
    E::store(Kh + t * HD + 2 * tid, kr0);
    E::store(Kh + t * HD + 2 * tid + 1, kr1);
    E::store(Vh + t * HD + 2 * tid, v0);
    E::store(Vh + t * HD + 2 * tid + 1, v1);
  }
  __syncthreads();

  // ---- pass 1: scores, one position per thread per sweep. Position t (index n-1) is scored from
  // the rotated key in LDS by thread 0; the cache row this launch writes is never read back.
  auto score = [&](const uint4 (&w)[KCH]) {
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const uint32_t ws[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
      const int e = c * VE;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          dot += qs[e + 2 * j] * __uint_as_float(ws[j] << 16) + qs[e + 2 * j + 1] * __uint_as_float(ws[j] & 0xffff0000u);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) dot += qs[e + j] * __uint_as_float(ws[j]);
      }
    }
    return Elem<T>::round(Elem<T>::round(dot) / a.scale);
  };
  float mx = -INFINITY;
#pragma unroll
  for (int q = 0; q < KP; ++q) {
    const int i = tid + q * kThreads;
    const float s0 = score(krow[q]);
    if (i < nc) {
      sc[i] = s0;
      mx = fmaxf(mx, s0);
    }
  }
  for (int i = tid + KP * kThreads; i < nc; i += kThreads) {   // spans longer than the prefetch
#pragma unroll
    for (int c = 0; c < KCH; ++c) krow[0][c] = reinterpret_cast<const uint4*>(Kh + (int64_t)(lo + i) * HD)[c];
    const float s1 = score(krow[0]);
    sc[i] = s1;
    mx = fmaxf(mx, s1);
  }
  if (tid == 0) {
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < HD; ++e) dot += qs[e] * ks[e];
    const float s2 = Elem<T>::round(Elem<T>::round(dot) / a.scale);
    sc[n - 1] = s2;
    mx = fmaxf(mx, s2);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, red[w]);
  __syncthreads();                                     // red is reused below
  float sum = 0.f;
  for (int i = tid; i < n; i += kThreads) {
    const float p = __expf(sc[i] - M);
    sc[i] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) L += red[w];

  // ---- pass 2: y = sum_j p_j V[j]. Wave w owns cached positions [j0, j1); a load instruction
  // covers RPI whole rows, lane -> (row slot, 16-byte chunk); the first CH chunks are in flight.
  float acc[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) acc[e] = 0.f;
  auto accumulate = [&](const uint4& w, int i) {
    if (i >= j1) return;                               // a clamped row: never folded in, even as 0 * x
    const float p = Elem<T>::round(sc[i] / L);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += p * __uint_as_float(ws[j] << 16);
        acc[2 * j + 1] += p * __uint_as_float(ws[j] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += p * __uint_as_float(ws[j]);
    }
  };
#pragma unroll
  for (int u = 0; u < CH; ++u) accumulate(vrow[u], j0 + u * RPI + slot);
  for (int i0 = j0 + CH * RPI; i0 < j1; i0 += CH * RPI) {   // blocks longer than CH instructions
#pragma unroll
    for (int u = 0; u < CH; ++u)
      vrow[u] = reinterpret_cast<const uint4*>(Vh + (int64_t)(lo + min(i0 + u * RPI + slot, ck)) * HD)[dg];
#pragma unroll
    for (int u = 0; u < CH; ++u) accumulate(vrow[u], i0 + u * RPI + slot);
  }
  // sum the RPI row slots of the wave (lanes dg, dg + LPR, ...), then the 16 waves in LDS
#pragma unroll
  for (int e = 0; e < VE; ++e) {
    float v = acc[e];
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) v += __shfl_xor(v, off);
    acc[e] = v;
  }
  if (slot == 0) {
#pragma unroll
    for (int e = 0; e < VE; ++e) part[wave][dg * VE + e] = acc[e];
  }
  __syncthreads();
  if (tid < HD) {
    float s = Elem<T>::round(sc[n - 1] / L) * vs[tid];      // position t
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += part[w][tid];
    Elem<T>::store((T*)a.y + (int64_t)b * a.y_bstride + (int64_t)h * HD + tid, s);
  }
}

template <typename T>
int launch(const AttnArgs& a, int B, int hd, hipStream_t s) {
  const int nmax = a.window > 0 ? min(a.window, a.Tmax) : a.Tmax;
  const size_t lds = (size_t)nmax * sizeof(float);
  dim3 grid(a.H, B), block(kThreads);
  switch (hd) {
    case 16: decode_attention_kernel<T, 16><<<grid, block, lds, s>>>(a); break;
    case 32: decode_attention_kernel<T, 32><<<grid, block, lds, s>>>(a); break;
    case 64: decode_attention_kernel<T, 64><<<grid, block, lds, s>>>(a); break;
    default: decode_attention_kernel<T, 128><<<grid, block, lds, s>>>(a); break;
  }
  return dh_check_launch("dh_decode_attention");
}

// ---------------------------------------------------------------------------------------------
// Split-window form for small batches (dh_decode_attention_split): the window is cut into S
// segments and each (segment, head, row) gets its own workgroup, so a head's keys and values
// stream through S compute units instead of one (the single-workgroup kernel above is bound by one
// CU's request rate at batch 1). Segment s computes, over its positions, the rounded scores, their
// maximum m_s, l_s = sum exp(s_j - m_s) and the unnormalised value sum o_s = sum exp(s_j - m_s)
// V_j (fp32), into a caller-provided workspace; a second launch combines the S records of a head:
//   M = max_s m_s,  y = round( sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s ).
// Same scores (rounded where the eager step rounds them) and the same softmax; the probabilities
// enter the value sum in fp32 (the single-workgroup kernel rounds them to the model dtype first,
// as the eager bf16 step does). The segment holding t rotates k, writes the cache row of t and
// takes position t from LDS, never from the cache.
// ---------------------------------------------------------------------------------------------
constexpr int kSThreads = 128;
constexpr int kSplits = 16;
constexpr int kMaxSplitPos = kMaxWindow / kSplits;    // positions per segment (LDS scores)

template <typename T, int HD>
__global__ __launch_bounds__(kSThreads) void decode_attention_split_kernel(AttnArgs a, int S, float* ws) {
  __shared__ float qs[HD], ks[HD], vsh[HD];
  __shared__ float sc[kMaxSplitPos];
  __shared__ float red[kSThreads / 64];
  __shared__ float part[kSThreads / 64][HD];
  constexpr int VE = 16 / (int)sizeof(T);             // elements per 16-byte chunk
  constexpr int KCH = HD / VE;                        // chunks per cache row
  constexpr int RPI = 64 / KCH;                       // rows per wave instruction in the value pass
  constexpr int NW = kSThreads / 64;
  constexpr int VCH = 8;                              // value instructions in flight per lane
  const int sg = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t = load_uniform(a.t_dev);
  if (t < 0 || t >= a.Tmax) return;                   // workgroup-uniform: nothing to do
  const int lo = a.window > 0 ? (int)max((int64_t)0, t + 1 - a.window) : 0;
  const int n = (int)t - lo + 1;                      // positions lo .. t; index n-1 is t itself
  const int P = (n + S - 1) / S;
  const int j0 = min(sg * P, n), j1 = min(n, j0 + P); // this segment's indices [j0, j1)
  const bool has_t = j0 <= n - 1 && n - 1 < j1;
  const int jc1 = min(j1, n - 1);                     // cached indices [j0, jc1)
  const int64_t head_off = ((int64_t)b * a.H + h) * a.Tmax * HD;
  T* Kh = (T*)a.K + head_off;
  T* Vh = (T*)a.V + head_off;

  // ---- rotation operands first (raw bits, every thread, clamped index), then the first key row of
  // this thread and the first value block, then the rotation
  const bool roper = tid < HD / 2;
  uint32_t rop[8];
  {
    const int pt = min(tid, HD / 2 - 1);
    const int64_t base = (int64_t)b * a.qkv_bstride + (int64_t)h * HD + 2 * pt;
    rop[0] = raw_load((const T*)a.cos + t * (HD / 2) + pt);
    rop[1] = raw_load((const T*)a.sin + t * (HD / 2) + pt);
    rop[2] = raw_load((const T*)a.q + base);
    rop[3] = raw_load((const T*)a.q + base + 1);
    rop[4] = raw_load((const T*)a.k + base);
    rop[5] = raw_load((const T*)a.k + base + 1);
    rop[6] = raw_load((const T*)a.v + base);
    rop[7] = raw_load((const T*)a.v + base + 1);
  }
  DH_ISSUE_FENCE();
  // only this segment's cached rows are requested (a segment is often shorter than one sweep)
  uint4 krow[KCH];
  {
    const int i = j0 + tid;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      krow[c] = make_uint4(0u, 0u, 0u, 0u);
      if (i < jc1) krow[c] = reinterpret_cast<const uint4*>(Kh + (int64_t)(lo + i) * HD)[c];
    }
  }
  const int slot = lane / KCH, dg = lane % KCH;
  uint4 vrow[VCH];
#pragma unroll
  for (int u = 0; u < VCH; ++u) {
    const int i = j0 + (u * NW + wave) * RPI + slot;
    vrow[u] = make_uint4(0u, 0u, 0u, 0u);
    if (i < jc1) vrow[u] = reinterpret_cast<const uint4*>(Vh + (int64_t)(lo + i) * HD)[dg];
  }
  DH_ISSUE_FENCE();
  if (roper) {
    asm volatile("" : "+v"(rop[0]), "+v"(rop[1]), "+v"(rop[2]), "+v"(rop[3]), "+v"(rop[4]), "+v"(rop[5]),
                 "+v"(rop[6]), "+v"(rop[7]));           // converted here, after the key/value requests
    const float c = raw_f<T>(rop[0]), s = raw_f<T>(rop[1]);
    const float q0 = raw_f<T>(rop[2]), q1 = raw_f<T>(rop[3]);
    const float k0 = raw_f<T>(rop[4]), k1 = raw_f<T>(rop[5]);
    const float v0 = raw_f<T>(rop[6]), v1 = raw_f<T>(rop[7]);
    typedef Elem<T> E;
    float qr0, qr1, kr0, kr1;
    {
#pragma clang fp contract(off)
      qr0 = E::round(E::round(q0 * c) - E::round(q1 * s));
      qr1 = E::round(E::round(q0 * s) + E::round(q1 * c));
      kr0 = E::round(E::round(k0 * c) - E::round(k1 * s));
      kr1 = E::round(E::round(k0 * s) + E::round(k1 * c));
    }
    qs[2 * tid] = qr0; qs[2 * tid + 1] = qr1;
    ks[2 * tid] = kr0; ks[2 * tid + 1] = kr1;
    vsh[2 * tid] = v0; vsh[2 * tid + 1] = v1;
    if (has_t) {
      E::store(Kh + t * HD + 2 * tid, kr0);
      E::store(Kh + t * HD + 2 * tid + 1, kr1);
      E::store(Vh + t * HD + 2 * tid, v0);
      E::store(Vh + t * HD + 2 * tid + 1, v1);
    }
  }
  __syncthreads();

  // ---- scores of the cached positions (one per thread per sweep) and of t (thread 0, from LDS)
  auto score = [&](const uint4 (&w)[KCH]) {
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const uint32_t wsd[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
      const int e = c * VE;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          dot += qs[e + 2 * j] * __uint_as_float(wsd[j] << 16) + qs[e + 2 * j + 1] * __uint_as_float(wsd[j] & 0xffff0000u);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) dot += qs[e + j] * __uint_as_float(wsd[j]);
      }
    }
    return Elem<T>::round(Elem<T>::round(dot) / a.scale);
  };
  float mx = -INFINITY;
  for (int i0 = j0; i0 < jc1; i0 += kSThreads) {
    const int i = i0 + tid;
    if (i0 > j0 && i < jc1) {                          // sweeps past the first (long segments)
#pragma unroll
      for (int c = 0; c < KCH; ++c) krow[c] = reinterpret_cast<const uint4*>(Kh + (int64_t)(lo + i) * HD)[c];
    }
    const float s0 = score(krow);
    if (i < jc1) {
      sc[i - j0] = s0;
      mx = fmaxf(mx, s0);
    }
  }
  if (has_t && tid == 0) {
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < HD; ++e) dot += qs[e] * ks[e];
    const float s2 = Elem<T>::round(Elem<T>::round(dot) / a.scale);
    sc[n - 1 - j0] = s2;
    mx = fmaxf(mx, s2);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, red[w]);
  __syncthreads();                                     // red is reused below
  float sum = 0.f;
  for (int i = j0 + tid; i < j1; i += kSThreads) {
    const float p = __expf(sc[i - j0] - M);
    sc[i - j0] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  float Ls = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) Ls += red[w];

  // ---- o = sum_i p_i V_i over the cached positions (lane -> (row slot, chunk)), then position t
  float acc[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) acc[e] = 0.f;
  auto accumulate = [&](const uint4& w, int i) {
    if (i >= jc1) return;                              // a row outside the segment: never folded in
    const float p = sc[i - j0];
    const uint32_t wsd[4] = {w.x, w.y, w.z, w.w};
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += p * __uint_as_float(wsd[j] << 16);
        acc[2 * j + 1] += p * __uint_as_float(wsd[j] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += p * __uint_as_float(wsd[j]);
    }
  };
#pragma unroll
  for (int u = 0; u < VCH; ++u) accumulate(vrow[u], j0 + (u * NW + wave) * RPI + slot);
  for (int i0 = j0 + VCH * NW * RPI; i0 < jc1; i0 += VCH * NW * RPI) {   // segments past the prefetch
#pragma unroll
    for (int u = 0; u < VCH; ++u) {
      const int i = i0 + (u * NW + wave) * RPI + slot;
      if (i < jc1) vrow[u] = reinterpret_cast<const uint4*>(Vh + (int64_t)(lo + i) * HD)[dg];
    }
#pragma unroll
    for (int u = 0; u < VCH; ++u) accumulate(vrow[u], i0 + (u * NW + wave) * RPI + slot);
  }
#pragma unroll
  for (int e = 0; e < VE; ++e) {
    float v = acc[e];
#pragma unroll
    for (int off = KCH; off < 64; off <<= 1) v += __shfl_xor(v, off);
    acc[e] = v;
  }
  if (slot == 0) {
#pragma unroll
    for (int e = 0; e < VE; ++e) part[wave][dg * VE + e] = acc[e];
  }
  __syncthreads();
  float* rec = ws + (((int64_t)b * a.H + h) * S + sg) * (2 + HD);
  if (tid < HD) {
    float o = has_t ? sc[n - 1 - j0] * vsh[tid] : 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) o += part[w][tid];
    rec[2 + tid] = o;
  }
  if (tid == 0) {
    rec[0] = M;                                         // -inf for an empty segment
    rec[1] = Ls;
  }
}

template <typename T, int HD>
__global__ __launch_bounds__(HD) void decode_attention_combine_kernel(AttnArgs a, int S, const float* ws) {
  const int h = blockIdx.x, b = blockIdx.y, e = threadIdx.x;
  const int64_t t = load_uniform(a.t_dev);
  if (t < 0 || t >= a.Tmax) return;
  const float* rec = ws + ((int64_t)b * a.H + h) * S * (2 + HD);
  // every record requested before any is used (a loop over S would wait once per record)
  float m[kSplits], l[kSplits], o[kSplits];
#pragma unroll
  for (int s = 0; s < kSplits; ++s) {
    const float* r = rec + min(s, S - 1) * (2 + HD);
    m[s] = r[0];
    l[s] = r[1];
    o[s] = r[2 + e];
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kSplits; ++s) M = s < S ? fmaxf(M, m[s]) : M;
  float L = 0.f, y = 0.f;
#pragma unroll
  for (int s = 0; s < kSplits; ++s) {
    const float w = (s < S && m[s] > -INFINITY) ? __expf(m[s] - M) : 0.f;
    L += w * l[s];
    y += w * o[s];
  }
  Elem<T>::store((T*)a.y + (int64_t)b * a.y_bstride + (int64_t)h * HD + e, y / L);
}

template <typename T>
int launch_split(const AttnArgs& a, int B, int hd, int S, float* ws, hipStream_t s) {
  dim3 g1(S, a.H, B), g2(a.H, B);
  switch (hd) {
    case 16:
      decode_attention_split_kernel<T, 16><<<g1, kSThreads, 0, s>>>(a, S, ws);
      decode_attention_combine_kernel<T, 16><<<g2, 16, 0, s>>>(a, S, ws);
      break;
    case 32:
      decode_attention_split_kernel<T, 32><<<g1, kSThreads, 0, s>>>(a, S, ws);
      decode_attention_combine_kernel<T, 32><<<g2, 32, 0, s>>>(a, S, ws);
      break;
    case 64:
      decode_attention_split_kernel<T, 64><<<g1, kSThreads, 0, s>>>(a, S, ws);
      decode_attention_combine_kernel<T, 64><<<g2, 64, 0, s>>>(a, S, ws);
      break;
    default:
      decode_attention_split_kernel<T, 128><<<g1, kSThreads, 0, s>>>(a, S, ws);
      decode_attention_combine_kernel<T, 128><<<g2, 128, 0, s>>>(a, S, ws);
      break;
  }
  return dh_check_launch("dh_decode_attention_split");
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

extern "C" int dh_decode_attention(int dtype, const void* q, const void* k, const void* v, int64_t qkv_bstride,
                                   const void* rope_cos, const void* rope_sin, void* K_cache, void* V_cache,
                                   const int64_t* t_dev, void* y, int64_t y_bstride, int B, int H, int hd,
                                   int Tmax, int window, void* stream) {
  const char* who = "dh_decode_attention";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && H >= 1 && Tmax >= 1 && window >= 0, DH_ERR_INVALID_ARG,
             "%s: B=%d H=%d Tmax=%d window=%d", who, B, H, Tmax, window);
  DH_REQUIRE(hd == 16 || hd == 32 || hd == 64 || hd == 128, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: hd=%d not in {16,32,64,128}", who, hd);
  const int nmax = window > 0 ? (window < Tmax ? window : Tmax) : Tmax;
  DH_REQUIRE(nmax <= kMaxWindow, DH_ERR_UNSUPPORTED_SHAPE, "%s: attention span %d exceeds %d", who, nmax,
             kMaxWindow);
  DH_REQUIRE(q && k && v && rope_cos && rope_sin && K_cache && V_cache && t_dev && y, DH_ERR_INVALID_ARG,
             "%s: null pointer argument", who);
  DH_REQUIRE(aligned(K_cache, 16) && aligned(V_cache, 16), DH_ERR_INVALID_ARG, "%s: caches need 16-byte alignment",
             who);
  AttnArgs a{q, k, v, qkv_bstride, rope_cos, rope_sin, K_cache, V_cache, t_dev, y, y_bstride, H, Tmax, window,
             sqrtf((float)hd)};
  hipStream_t s = (hipStream_t)stream;
  return dtype == DH_BF16 ? launch<bf16_t>(a, B, hd, s) : launch<float>(a, B, hd, s);
}

extern "C" int64_t dh_decode_attention_workspace_bytes(int B, int H, int hd) {
  return (int64_t)B * H * kSplits * (2 + hd) * (int64_t)sizeof(float);
}

extern "C" int dh_decode_attention_split(int dtype, const void* q, const void* k, const void* v, int64_t qkv_bstride,
                                         const void* rope_cos, const void* rope_sin, void* K_cache, void* V_cache,
                                         const int64_t* t_dev, void* y, int64_t y_bstride, int B, int H, int hd,
                                         int Tmax, int window, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
  const char* who = "dh_decode_attention_split";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && B <= 65535 && H >= 1 && H <= 65535 && Tmax >= 1 && window >= 0, DH_ERR_INVALID_ARG,
             "%s: B=%d H=%d Tmax=%d window=%d", who, B, H, Tmax, window);
  DH_REQUIRE(hd == 16 || hd == 32 || hd == 64 || hd == 128, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: hd=%d not in {16,32,64,128}", who, hd);
  const int nmax = window > 0 ? (window < Tmax ? window : Tmax) : Tmax;
  DH_REQUIRE(nmax <= kMaxWindow, DH_ERR_UNSUPPORTED_SHAPE, "%s: attention span %d exceeds %d", who, nmax,
             kMaxWindow);
  DH_REQUIRE(q && k && v && rope_cos && rope_sin && K_cache && V_cache && t_dev && y && workspace,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(aligned(K_cache, 16) && aligned(V_cache, 16) && aligned(workspace, 16), DH_ERR_INVALID_ARG,
             "%s: caches and workspace need 16-byte alignment", who);
  DH_REQUIRE(workspace_bytes >= dh_decode_attention_workspace_bytes(B, H, hd), DH_ERR_INVALID_ARG,
             "%s: workspace of %lld bytes, needs %lld", who, (long long)workspace_bytes,
             (long long)dh_decode_attention_workspace_bytes(B, H, hd));
  AttnArgs a{q, k, v, qkv_bstride, rope_cos, rope_sin, K_cache, V_cache, t_dev, y, y_bstride, H, Tmax, window,
             sqrtf((float)hd)};
  const int S = nmax < kSplits ? nmax : kSplits;
  hipStream_t s = (hipStream_t)stream;
  return dtype == DH_BF16 ? launch_split<bf16_t>(a, B, hd, S, (float*)workspace, s)
                          : launch_split<float>(a, B, hd, S, (float*)workspace, s);
}
