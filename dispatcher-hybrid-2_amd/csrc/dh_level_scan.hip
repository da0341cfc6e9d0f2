// Parallel level scan with the gate activations fused in, for gfx950.
//
// Semantics (reference dispatcher_hybrid/modeling_dispatcher.py:86-88, 111-121):
//   M[b,t,l] = [t >= 2^l] * (mask ? [mask[b,t,l] > 0] : 1)
//   a = sigmoid(pre_i) * M ; f = sigmoid(pre_f) * M + (1 - M) ; r = sigmoid(pre_r)
//   V = V0 ; for l < n_lv:  V[t] <- f[t,l] * V[t] + a[t,l] * r[t-2^l,l] * V[t-2^l]
// Every level reads the previous level's state, so a position's update needs the whole column of
// the previous level. The reference's roll() wraps future rows into t < 2^l and cancels them with
// a = 0; here those reads are predicated away, which gives the same result for finite data.
// With `activated` the gate inputs are already a, f and r (dh_gate_preacts_fwd with `activate`):
// then a = 0 and f = 1 wherever M = 0, so every position takes the update unpredicated.
//
// Work decomposition: one workgroup (8 wave64s) per (batch row b, head h, chunk of C columns of
// the head's hd). The chunk's state for all T positions lives in registers (PPT positions per
// thread, position t = tid + j*512) and each level exchanges r*V through an LDS column of T*C fp32
// (128 KB at T = 4096, C = 8), two barriers per level. Gate and mask reads go through element
// strides; with the head-major gate layout (unit stride in t) a wave's 64 consecutive positions
// read one contiguous 128-byte line per gate. The next level's gates are requested before the
// current level's exchange (barriers here wait for LDS only, not for global loads), so their
// latency hides behind it. The hd/C chunk workgroups of one (b, h) read the same V0 cache lines and
// the same gates, so they are given the same blockIdx % 8 (one XCD under round-robin dispatch) and
// consecutive dispatch slots, so those lines are fetched once into that XCD's L2.
#include "dh_common.h"

#include <type_traits>

namespace {

constexpr int kThreads = 512;

enum { kPreNoMask = 0, kPreMask = 1, kActivated = 2 };

struct ScanArgs {
  const void* pre_i;
  const void* pre_f;
  const void* pre_r;
  int64_t spb, spt, spl, sph;
  const void* mask;
  int64_t smb, smt, sml;
  const void* V0;
  int64_t svb, svt;
  void* V;
  void* ring;              // nullable decoder ring buffer (b, S, H*hd), S = 2^(ring_L+1) - 2
  int b, T, H, hd, n_lv, ring_L;
};

// raw element bits, converted after the loads of a burst have all been issued
template <typename T> struct Raw;
template <> struct Raw<bf16_t> {
  __device__ __forceinline__ static uint32_t load(const bf16_t* p) { return *p; }
  __device__ __forceinline__ static float f(uint32_t r) { return __uint_as_float(r << 16); }
};
template <> struct Raw<float> {
  __device__ __forceinline__ static uint32_t load(const float* p) { return __float_as_uint(*p); }
  __device__ __forceinline__ static float f(uint32_t r) { return __uint_as_float(r); }
};

// The C columns of one position as ONE unconditional vector access (C*sizeof(T) bytes, aligned to
// that size: the host checks row strides and base pointers).
template <typename T, int C>
__device__ __forceinline__ void load_cols(const T* p, float (&v)[C]) {
  if constexpr (sizeof(T) == 2 && C == 1) {
    v[0] = bf16_to_f32(*p);
  } else {
    constexpr int NW = C * (int)sizeof(T) / 4;
    uint32_t w[NW];
    if constexpr (NW >= 4) {
#pragma unroll
      for (int q = 0; q < NW / 4; ++q) {
        const uint4 x = reinterpret_cast<const uint4*>(p)[q];
        w[4 * q] = x.x; w[4 * q + 1] = x.y; w[4 * q + 2] = x.z; w[4 * q + 3] = x.w;
      }
    } else if constexpr (NW == 2) {
      const uint2 x = *reinterpret_cast<const uint2*>(p);
      w[0] = x.x; w[1] = x.y;
    } else {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      if constexpr (sizeof(T) == 2) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        v[i] = __uint_as_float(w[i]);
      }
    }
  }
}

template <typename T, int C>
__device__ __forceinline__ void store_cols(T* p, const float (&v)[C]) {
  if constexpr (sizeof(T) == 2 && C == 1) {
    *p = f32_to_bf16(v[0]);
  } else {
    constexpr int NW = C * (int)sizeof(T) / 4;
    uint32_t w[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      if constexpr (sizeof(T) == 2)
        w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
      else
        w[i] = __float_as_uint(v[i]);
    }
    if constexpr (NW >= 4) {
#pragma unroll
      for (int q = 0; q < NW / 4; ++q)
        reinterpret_cast<uint4*>(p)[q] = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    } else if constexpr (NW == 2) {
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    } else {
      *reinterpret_cast<uint32_t*>(p) = w[0];
    }
  }
}

template <typename T, int C, int PPT, int MODE>
__global__ __launch_bounds__(kThreads) void level_scan_kernel(ScanArgs a) {
  __shared__ float rv[C * PPT * kThreads];
  // a whole level of raw gates in flight costs 4*PPT registers; past 32 positions per thread the
  // gates are fetched at the top of their own level instead
  constexpr bool kPrefetch = PPT <= 32;
  const int nchunks = a.hd / C;
  const int ngroups = a.b * a.H;
  const int bid = blockIdx.x;
  const int x = bid & 7, rem = bid >> 3;
  const int c = rem % nchunks, g = (rem / nchunks) * 8 + x;
  if (g >= ngroups) return;
  const int b = g / a.H, h = g % a.H;
  const int64_t col0 = (int64_t)h * a.hd + (int64_t)c * C;
  const int tid = threadIdx.x;

  const int64_t gb = (int64_t)b * a.spb + (int64_t)h * a.sph;
  const T* pi = (const T*)a.pre_i + gb;
  const T* pf = (const T*)a.pre_f + gb;
  const T* pr = (const T*)a.pre_r + gb;
  const T* mk = (const T*)a.mask + (MODE == kPreMask ? (int64_t)b * a.smb : 0);

  // V0: one unconditional vector load per position from the clamped row, zeroed past T afterwards
  float V[PPT][C];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int t = tid + j * kThreads;
    const int tc = t < a.T ? t : a.T - 1;
    load_cols<T, C>((const T*)a.V0 + (int64_t)b * a.svb + (int64_t)tc * a.svt + col0, V[j]);
  }
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const bool live = tid + j * kThreads < a.T;
#pragma unroll
    for (int cc = 0; cc < C; ++cc) V[j][cc] = live ? V[j][cc] : 0.f;
  }

  // per-position element offsets along t, shared by the three gates (32-bit: the host checks
  // (T-1)*stride fits); the per-level part of each address is a uniform base
  uint32_t goff[PPT], moff[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int t = tid + j * kThreads;
    const uint32_t tc = t < a.T ? t : a.T - 1;
    goff[j] = tc * (uint32_t)a.spt;
    moff[j] = tc * (uint32_t)a.smt;
  }
  uint32_t ri[PPT], rf[PPT], rr[PPT], rm[PPT];
  auto fetch = [&](int l) {
    const T* li = pi + (int64_t)l * a.spl;
    const T* lf = pf + (int64_t)l * a.spl;
    const T* lr = pr + (int64_t)l * a.spl;
    const T* lm = mk + (int64_t)l * a.sml;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      ri[j] = Raw<T>::load(li + goff[j]);
      rf[j] = Raw<T>::load(lf + goff[j]);
      rr[j] = Raw<T>::load(lr + goff[j]);
      if (MODE == kPreMask) rm[j] = Raw<T>::load(lm + moff[j]);
    }
  };
  if (kPrefetch) fetch(0);

  // decoder prefill: the state entering level j of the positions ring j still holds (the last
  // 2^(j+1)), at slot 2^(j+1) - 2 + (t & (2^(j+1) - 1)) (reference decoding.py:50-76, 143-185)
  const int64_t d = (int64_t)a.H * a.hd;
  auto write_slab = [&](int j) {
    if (a.ring == nullptr || j >= a.ring_L) return;   // uniform
    const int p0 = a.T - (2 << j);
    const int msk = (2 << j) - 1;
    T* rb = (T*)a.ring + (int64_t)b * ((int64_t)(2 << a.ring_L) - 2) * d + (int64_t)((2 << j) - 2) * d + col0;
#pragma unroll
    for (int jj = 0; jj < PPT; ++jj) {
      const int t = tid + jj * kThreads;
      if (t < a.T && t >= p0) store_cols<T, C>(rb + (int64_t)(t & msk) * d, V[jj]);
    }
  };
  write_slab(0);

  for (int l = 0; l < a.n_lv; ++l) {
    const int shift = 1 << l;
    if (!kPrefetch) fetch(l);
    // a position that takes no update at this level gets a = 0, f = 1 (as the activated inputs
    // already have it), so the update below runs unpredicated: f*V + 0*msg = V for finite data
    float rg[PPT], ad[PPT], fg[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int t = tid + j * kThreads;
      if (MODE == kActivated) {
        ad[j] = Raw<T>::f(ri[j]);
        fg[j] = Raw<T>::f(rf[j]);
        rg[j] = Raw<T>::f(rr[j]);
      } else {
        const bool up = t >= shift && (MODE != kPreMask || Raw<T>::f(rm[j]) > 0.f);
        ad[j] = up ? dh_sigmoid(Raw<T>::f(ri[j])) : 0.f;
        fg[j] = up ? dh_sigmoid(Raw<T>::f(rf[j])) : 1.f;
        rg[j] = dh_sigmoid(Raw<T>::f(rr[j]));
      }
    }
    if (kPrefetch) fetch(l + 1 < a.n_lv ? l + 1 : l);   // next level's gates fly during the exchange
    // r * V at every position (the message a level-l destination reads at lag 2^l); positions past
    // T are written but never read (every source t - 2^l of a position t < T is below T)
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int t = tid + j * kThreads;
#pragma unroll
      for (int cc = 0; cc < C; ++cc) rv[t * C + cc] = rg[j] * V[j][cc];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int t = tid + j * kThreads;
      const int s = t >= shift ? t - shift : 0;
#pragma unroll
      for (int cc = 0; cc < C; ++cc) V[j][cc] = fg[j] * V[j][cc] + ad[j] * rv[s * C + cc];
    }
    write_slab(l + 1);
    __syncthreads();
  }
  for (int j = a.n_lv + 1; j < a.ring_L; ++j) write_slab(j);   // beyond the horizon: passed through

#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int t = tid + j * kThreads;
    if (t < a.T) store_cols<T, C>((T*)a.V + ((int64_t)b * a.T + t) * ((int64_t)a.H * a.hd) + col0, V[j]);
  }
}

// Contexts up to 4096 positions: 1024 threads (PPT <= 4 positions each, 4 waves per SIMD) and
// C = 8 columns per workgroup. Each level exchanges the state itself, not r * V: position t
// publishes V[t] (column pairs as float2, consecutive positions in consecutive 8-byte words, so
// neither the writes nor the shifted reads conflict on LDS banks) and r[t] once, and the
// destination forms coef = a[t] * r[t - 2^l] once per position, then V = f * V + coef * V_src:
// two VALU operations per element and level instead of three. 144 KB of LDS at T = 4096.
template <typename T, int C, int PPT, int MODE>
__global__ __launch_bounds__(1024) void level_scan_wide_kernel(ScanArgs a) {
  constexpr int NT = 1024, TC = PPT * NT;
  // Double-buffered when two copies fit the 160 KB of LDS (T <= 2048): level l exchanges through
  // buffer l % 2, so the barrier after its reads is not needed (the next level writes the other
  // buffer, and a buffer is written again only after the following level's barrier). T = 2048:
  // 15.4 -> 14.0 us per launch. At T = 4096 (144 KB) one buffer and two barriers per level.
  constexpr int NB = (TC * (C * 4 + 4) * 2 <= 160 * 1024) ? 2 : 1;
  __shared__ float2 vs_[NB][C / 2][TC];
  __shared__ float rs_[NB][TC];
  const int nchunks = a.hd / C;
  const int ngroups = a.b * a.H;
  const int bid = blockIdx.x;
  const int x = bid & 7, rem = bid >> 3;
  const int c = rem % nchunks, g = (rem / nchunks) * 8 + x;
  if (g >= ngroups) return;
  const int b = g / a.H, h = g % a.H;
  const int64_t col0 = (int64_t)h * a.hd + (int64_t)c * C;
  const int tid = threadIdx.x;

  const int64_t gb = (int64_t)b * a.spb + (int64_t)h * a.sph;
  const T* pi = (const T*)a.pre_i + gb;
  const T* pf = (const T*)a.pre_f + gb;
  const T* pr = (const T*)a.pre_r + gb;
  const T* mk = (const T*)a.mask + (MODE == kPreMask ? (int64_t)b * a.smb : 0);

  float V[PPT][C];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int t = tid + j * NT;
    const int tc = t < a.T ? t : a.T - 1;
    load_cols<T, C>((const T*)a.V0 + (int64_t)b * a.svb + (int64_t)tc * a.svt + col0, V[j]);
  }
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const bool live = tid + j * NT < a.T;
#pragma unroll
    for (int cc = 0; cc < C; ++cc) V[j][cc] = live ? V[j][cc] : 0.f;
  }
  uint32_t goff[PPT], moff[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int t = tid + j * NT;
    const uint32_t tc = t < a.T ? t : a.T - 1;
    goff[j] = tc * (uint32_t)a.spt;
    moff[j] = tc * (uint32_t)a.smt;
  }
  struct GSet { uint32_t i[PPT], f[PPT], r[PPT], m[PPT]; };
  auto fetch = [&](int l, GSet& g) {
    const T* li = pi + (int64_t)l * a.spl;
    const T* lf = pf + (int64_t)l * a.spl;
    const T* lr = pr + (int64_t)l * a.spl;
    const T* lm = mk + (int64_t)l * a.sml;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      g.i[j] = Raw<T>::load(li + goff[j]);
      g.f[j] = Raw<T>::load(lf + goff[j]);
      g.r[j] = Raw<T>::load(lr + goff[j]);
      if (MODE == kPreMask) g.m[j] = Raw<T>::load(lm + moff[j]);
    }
  };
  // Two register sets of gates: level l reads set l % 2, then requests level l + 2 into it, so a
  // level's gates are in flight for two levels of work (one level ahead left the loads' round trip
  // exposed: T = 1024 9.0 -> 8.0 us per launch; three or four sets measured slower, C5 143 / 194 us
  // against 120, from the registers they take).
  GSet gs0, gs1;
  fetch(0, gs0);
  fetch(min(1, a.n_lv - 1), gs1);

  const int64_t d = (int64_t)a.H * a.hd;
  auto write_slab = [&](int j) {
    if (a.ring == nullptr || j >= a.ring_L) return;   // uniform
    const int p0 = a.T - (2 << j);
    const int msk = (2 << j) - 1;
    T* rb = (T*)a.ring + (int64_t)b * ((int64_t)(2 << a.ring_L) - 2) * d + (int64_t)((2 << j) - 2) * d + col0;
#pragma unroll
    for (int jj = 0; jj < PPT; ++jj) {
      const int t = tid + jj * NT;
      if (t < a.T && t >= p0) store_cols<T, C>(rb + (int64_t)(t & msk) * d, V[jj]);
    }
  };
  write_slab(0);

  auto level = [&](int l, GSet& g) {
    const uint32_t (&ri)[PPT] = g.i;
    const uint32_t (&rf)[PPT] = g.f;
    const uint32_t (&rr)[PPT] = g.r;
    const uint32_t (&rm)[PPT] = g.m;
    const int shift = 1 << l;
    float rg[PPT], ad[PPT], fg[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int t = tid + j * NT;
      if (MODE == kActivated) {
        ad[j] = Raw<T>::f(ri[j]);
        fg[j] = Raw<T>::f(rf[j]);
        rg[j] = Raw<T>::f(rr[j]);
      } else {
        const bool up = t >= shift && (MODE != kPreMask || Raw<T>::f(rm[j]) > 0.f);
        ad[j] = up ? dh_sigmoid(Raw<T>::f(ri[j])) : 0.f;
        fg[j] = up ? dh_sigmoid(Raw<T>::f(rf[j])) : 1.f;
        rg[j] = dh_sigmoid(Raw<T>::f(rr[j]));
      }
    }
    fetch(min(l + 2, a.n_lv - 1), g);                  // two levels ahead, into the set just consumed
    if (shift >= NT) {                                   // uniform
      // lags of whole slots (2^l = K * NT): the source of position tid + j * NT is this thread's
      // slot j - K, so the level needs no exchange and no barrier. Slots update in descending order,
      // so slot j - K still holds the previous level's state. Without a source (j < K) a = 0, and
      // the clamped slot 0 stands in, as the exchange's clamped read of position 0 does.
      auto step = [&](auto kc) {
        constexpr int K = decltype(kc)::value;
#pragma unroll
        for (int j = PPT - 1; j >= 0; --j) {
          const int sj = j - K >= 0 ? j - K : 0;
          const float coef = ad[j] * rg[sj];
#pragma unroll
          for (int q = 0; q < C / 2; ++q) {
            const float w0 = V[sj][2 * q], w1 = V[sj][2 * q + 1];
            V[j][2 * q] = __builtin_fmaf(coef, w0, fg[j] * V[j][2 * q]);
            V[j][2 * q + 1] = __builtin_fmaf(coef, w1, fg[j] * V[j][2 * q + 1]);
          }
        }
      };
      const int k = shift / NT;
      if (k == 1) step(std::integral_constant<int, 1>{});
      else if (k == 2) step(std::integral_constant<int, 2>{});
      else step(std::integral_constant<int, PPT>{});   // k >= PPT: no position has a source
      write_slab(l + 1);
      return;
    }
    const int bsel = NB == 2 ? (l & 1) : 0;
    auto& vs = vs_[bsel];
    auto& rs = rs_[bsel];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int t = tid + j * NT;
#pragma unroll
      for (int q = 0; q < C / 2; ++q) vs[q][t] = make_float2(V[j][2 * q], V[j][2 * q + 1]);
      rs[t] = rg[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int t = tid + j * NT;
      const int s = t >= shift ? t - shift : 0;          // a = 0 where there is no source
      const float coef = ad[j] * rs[s];
#pragma unroll
      for (int q = 0; q < C / 2; ++q) {
        const float2 w = vs[q][s];
        // V = coef * w + f * V as one explicit FMA in both update paths (left to the compiler, the
        // contraction it picks differs between them)
        V[j][2 * q] = __builtin_fmaf(coef, w.x, fg[j] * V[j][2 * q]);
        V[j][2 * q + 1] = __builtin_fmaf(coef, w.y, fg[j] * V[j][2 * q + 1]);
      }
    }
    write_slab(l + 1);
    if (NB == 1) __syncthreads();
  };
  for (int l = 0; l < a.n_lv; l += 2) {
    level(l, gs0);
    if (l + 1 < a.n_lv) level(l + 1, gs1);                // uniform
  }
  for (int j = a.n_lv + 1; j < a.ring_L; ++j) write_slab(j);

#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    const int t = tid + j * NT;
    if (t < a.T) store_cols<T, C>((T*)a.V + ((int64_t)b * a.T + t) * ((int64_t)a.H * a.hd) + col0, V[j]);
  }
}

template <typename T, int PPT, int C>
void launch_wide_c(const ScanArgs& a, int mode, hipStream_t s) {
  const int nchunks = a.hd / C;
  const int grid = ((a.b * a.H + 7) / 8) * 8 * nchunks;
  auto go = [&](auto kern) { kern<<<dim3(grid), dim3(1024), 0, s>>>(a); };
  if (mode == kActivated) go(level_scan_wide_kernel<T, C, PPT, kActivated>);
  else if (mode == kPreMask) go(level_scan_wide_kernel<T, C, PPT, kPreMask>);
  else go(level_scan_wide_kernel<T, C, PPT, kPreNoMask>);
}

// 8 columns per workgroup; 4 when 8 would leave CUs without a workgroup (a short single-row
// prefill: b = 1, 16 heads x 64 gives 128). With enough workgroups, 4 columns (two workgroups per
// CU) measured slower.
template <typename T, int PPT>
void launch_wide(const ScanArgs& a, int mode, hipStream_t s) {
  if ((int64_t)a.b * a.H * (a.hd / 8) < 256) launch_wide_c<T, PPT, 4>(a, mode, s);
  else launch_wide_c<T, PPT, 8>(a, mode, s);
}

template <typename T, int C, int PPT>
void launch(const ScanArgs& a, int mode, hipStream_t s) {
  const int nchunks = a.hd / C;
  const int ngroups = a.b * a.H;
  const int grid = ((ngroups + 7) / 8) * 8 * nchunks;
  if (mode == kActivated)
    level_scan_kernel<T, C, PPT, kActivated><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  else if (mode == kPreMask)
    level_scan_kernel<T, C, PPT, kPreMask><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  else
    level_scan_kernel<T, C, PPT, kPreNoMask><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
}

template <typename T>
int dispatch(const ScanArgs& a, int mode, hipStream_t s) {
  if (a.T <= 1024) launch_wide<T, 1>(a, mode, s);
  else if (a.T <= 2048) launch_wide<T, 2>(a, mode, s);
  else if (a.T <= 4096) launch_wide<T, 4>(a, mode, s);
  else if (a.T <= 8192) launch<T, 4, 16>(a, mode, s);
  else if (a.T <= 16384) launch<T, 2, 32>(a, mode, s);
  else launch<T, 1, 64>(a, mode, s);
  return dh_check_launch("dh_level_scan_fwd");
}

}  // namespace

extern "C" int dh_level_scan_fwd(int dtype, const void* pre_i, const void* pre_f, const void* pre_r,
                                 int64_t stride_pb, int64_t stride_pt, int64_t stride_pl, int64_t stride_ph,
                                 const void* mask, int64_t stride_mb, int64_t stride_mt, int64_t stride_ml,
                                 const void* V0, int64_t stride_vb, int64_t stride_vt, void* V, int b, int T,
                                 int H, int hd, int n_lv, int activated, void* ring, int ring_L,
                                 void* stream) {
  const char* who = "dh_level_scan_fwd";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(b >= 1 && T >= 1, DH_ERR_INVALID_ARG, "%s: b=%d T=%d must be >= 1", who, b, T);
  DH_REQUIRE(T <= 32768, DH_ERR_UNSUPPORTED_SHAPE, "%s: T=%d exceeds 32768", who, T);
  DH_REQUIRE(H >= 1 && H <= 64, DH_ERR_UNSUPPORTED_SHAPE, "%s: H=%d not in [1,64]", who, H);
  DH_REQUIRE(hd == 16 || hd == 32 || hd == 64 || hd == 128, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: hd=%d not in {16,32,64,128}", who, hd);
  DH_REQUIRE(n_lv >= 1 && n_lv <= 16, DH_ERR_UNSUPPORTED_SHAPE, "%s: n_lv=%d not in [1,16]", who, n_lv);
  DH_REQUIRE(pre_i && pre_f && pre_r && V0 && V, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(stride_vt >= (int64_t)H * hd, DH_ERR_INVALID_ARG, "%s: V0 row stride %lld < H*hd", who,
             (long long)stride_vt);
  DH_REQUIRE(stride_pb >= 0 && stride_pt >= 0 && stride_pl >= 0 && stride_ph >= 0, DH_ERR_INVALID_ARG,
             "%s: negative gate stride", who);
  DH_REQUIRE((int64_t)(T - 1) * stride_pt < ((int64_t)1 << 31) && (int64_t)(T - 1) * stride_mt < ((int64_t)1 << 31),
             DH_ERR_UNSUPPORTED_SHAPE, "%s: (T-1) * gate/mask t-stride exceeds 2^31 elements", who);
  const int64_t esz = dtype == DH_BF16 ? 2 : 4;
  DH_REQUIRE((uintptr_t)V0 % 16 == 0 && (uintptr_t)V % 16 == 0 && (stride_vt * esz) % 16 == 0 &&
                 (stride_vb * esz) % 16 == 0,
             DH_ERR_INVALID_ARG, "%s: V0/V need 16-byte aligned rows", who);
  DH_REQUIRE(!ring || (ring_L >= n_lv && ring_L <= 16 && (uintptr_t)ring % 16 == 0), DH_ERR_INVALID_ARG,
             "%s: ring needs ring_L in [n_lv, 16] (got %d, n_lv %d) and 16-byte alignment", who, ring_L, n_lv);
  ScanArgs a{pre_i, pre_f, pre_r, stride_pb, stride_pt, stride_pl, stride_ph, mask, stride_mb, stride_mt,
             stride_ml, V0, stride_vb, stride_vt, V, ring, b, T, H, hd, n_lv, ring ? ring_L : 0};
  const int mode = activated ? kActivated : (mask ? kPreMask : kPreNoMask);
  hipStream_t s = (hipStream_t)stream;
  return dtype == DH_F32 ? dispatch<float>(a, mode, s) : dispatch<bf16_t>(a, mode, s);
}
