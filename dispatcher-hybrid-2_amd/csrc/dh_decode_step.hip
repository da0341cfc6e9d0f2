// Decode step of one tree layer (gates for every level + the level recurrence over the ring
// buffers) for gfx950.
//
// Semantics follow the reference per-token step (dispatcher_hybrid/fused_step.py:26-88,
// dispatcher_hybrid/decoding.py:187-222):
//   for l < L:  src = t - 2^l, ok = src >= 0, s = max(src, 0)
//               hid = relu(A + ok * B_hist[s])^2                       (fp32)
//               ig = sigmoid(Wi[l].hid + bi[l]) * ok
//               fg = sigmoid(Wf[l].hid + bf[l]) * ok + (1 - ok)
//               rg = sigmoid(Wr[l].hid + br[l])  -> rg_hist[t, l]      (model dtype)
//   V = V0 ; ring_0[slot(0, t)] = V0
//   for l < L:  V = fg_l * V + ig_l * ok * rg_hist[s, l] * ring_l[slot(l, s)]
//               if l + 1 < L: ring_{l+1}[slot(l+1, t)] = V
//   Y = V ;  slot(j, p) = 2^(j+1) - 2 + (p & (2^(j+1) - 1))
//
// Work decomposition of the fused kernel (MI355X: 256 CUs in 8 XCDs, wave64): one workgroup of
// 512 threads per (head h, block of batch rows); no workgroup depends on another, so the kernel
// needs no device-scope fences (which on gfx950 write back and invalidate the per-XCD L2s).
//   1. Every thread that owns a (row, element) of the recurrence prefetches its L ring sources and
//      transmit gates first: the slot written at t never aliases the slot read at t - 2^l, and
//      rg_hist rows t - 2^l < t are final, so these loads overlap the gate phase.
//   2. Gate readouts: the (level, 16-byte k-chunk) items of head h's 3*L weight rows are spread over
//      the threads; each item's three weight chunks are loaded once and applied to every row of the
//      block; partial dots are reduced across the lanes sharing a level with shuffles and
//      accumulated in LDS.
//   3. Sigmoid heads and masks, rg_hist[t] stores, then the L-level recurrence per (row, element),
//      all in registers, writing ring slots and Y.
// The separately launched halves (dh_step_gates: one workgroup per (head, level) over all rows;
// dh_step_scan: one workgroup per head) keep the reference's two-kernel buffer contract.
#include "dh_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxL = 16;
constexpr int kRowChunk = 8;          // batch rows reduced together per weight pass (split kernels)
constexpr int kFusedThreads = 1024;   // fused kernel workgroup (16 wave64s)
constexpr int kMaxHd = 128;

struct StepArgs {
  const void* A;
  const void* B_hist;
  const void* Wi;
  const void* Wf;
  const void* Wr;
  const void* bi;
  const void* bf;
  const void* br;
  const int64_t* t_dev;
  void* rg_hist;
  void* V_ring;
  const void* V0;
  void* Y;
  float* IG;
  float* FG;
  int B, Tmax, S, GH, H, hd, L;
  int rows_per_block;
};

__device__ __forceinline__ void block_coords(int bid, int H, int L, int& h, int& l) {
  if ((H & 7) == 0) {
    const int x = bid & 7, slot = bid >> 3;
    h = x + 8 * (slot / L);
    l = slot % L;
  } else {
    h = bid / L;
    l = bid % L;
  }
}

// Gate readouts of level l, head h for every batch row. Writes IG/FG [b][l][h] (fp32) and
// rg_hist[b, t, l, h] (model dtype).
template <typename T>
__device__ void gates_phase(const StepArgs& a, int h, int l, int64_t t) {
  __shared__ float part[kWaves][kRowChunk][3];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t src = t - ((int64_t)1 << l);
  const bool ok = src >= 0;
  const int64_t s = ok ? src : 0;
  const int64_t wrow = ((int64_t)l * a.H + h) * a.GH;
  const T* Wi = (const T*)a.Wi + wrow;
  const T* Wf = (const T*)a.Wf + wrow;
  const T* Wr = (const T*)a.Wr + wrow;

  for (int b0 = 0; b0 < a.B; b0 += kRowChunk) {
    const int nb = min(kRowChunk, a.B - b0);
    float acc[kRowChunk][3];
#pragma unroll
    for (int r = 0; r < kRowChunk; ++r) acc[r][0] = acc[r][1] = acc[r][2] = 0.f;

    for (int k = tid * 4; k < a.GH; k += kThreads * 4) {
      float wi[4], wf[4], wr[4];
      load4(Wi + k, wi);
      load4(Wf + k, wf);
      load4(Wr + k, wr);
#pragma unroll
      for (int r = 0; r < kRowChunk; ++r) {
        if (r < nb) {
          const int64_t b = b0 + r;
          float av[4], bv[4] = {0.f, 0.f, 0.f, 0.f};
          load4((const T*)a.A + b * a.GH + k, av);
          if (ok) load4((const T*)a.B_hist + (b * a.Tmax + s) * a.GH + k, bv);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float x = fmaxf(av[j] + bv[j], 0.f);
            x = x * x;
            acc[r][0] += wi[j] * x;
            acc[r][1] += wf[j] * x;
            acc[r][2] += wr[j] * x;
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kRowChunk; ++r) {
      if (r < nb) {
#pragma unroll
        for (int x = 0; x < 3; ++x) {
          const float v = wave_sum(acc[r][x]);
          if (lane == 0) part[wave][r][x] = v;
        }
      }
    }
    __syncthreads();
    if (tid < nb) {
      const int64_t b = b0 + tid;
      float p[3];
#pragma unroll
      for (int x = 0; x < 3; ++x) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += part[w][tid][x];
        p[x] = v;
      }
      const int64_t gi = (int64_t)l * a.H + h;
      const float okf = ok ? 1.f : 0.f;
      const float ig = dh_sigmoid(p[0] + Elem<T>::load((const T*)a.bi + gi)) * okf;
      const float fg = dh_sigmoid(p[1] + Elem<T>::load((const T*)a.bf + gi)) * okf + (1.f - okf);
      const float rg = dh_sigmoid(p[2] + Elem<T>::load((const T*)a.br + gi));
      const int64_t gw = (b * a.L + l) * a.H + h;
      a.IG[gw] = ig;
      a.FG[gw] = fg;
      Elem<T>::store((T*)a.rg_hist + ((b * a.Tmax + t) * a.L + l) * a.H + h, rg);
    }
    __syncthreads();
  }
}

// L-level recurrence of head h for every batch row, over the ring buffers.
template <typename T>
__device__ void scan_phase(const StepArgs& a, int h, int64_t t) {
  const int tid = threadIdx.x;
  const int64_t d = (int64_t)a.H * a.hd;
  const int rows_per_pass = kThreads / a.hd;
  const int e = tid % a.hd;
  for (int b = tid / a.hd; b < a.B; b += rows_per_pass) {
    T* ring = (T*)a.V_ring + (int64_t)b * a.S * d + (int64_t)h * a.hd + e;
    const T* rgb = (const T*)a.rg_hist + (int64_t)b * a.Tmax * a.L * a.H + h;
    const float* igb = a.IG + (int64_t)b * a.L * a.H + h;
    const float* fgb = a.FG + (int64_t)b * a.L * a.H + h;
    float vs[kMaxL], rgs[kMaxL], ig[kMaxL], fg[kMaxL];
#pragma unroll
    for (int l = 0; l < kMaxL; ++l) {
      if (l < a.L) {
        const int64_t src = t - ((int64_t)1 << l);
        const bool ok = src >= 0;
        vs[l] = ok ? Elem<T>::load(ring + (ring_offset(l) + (src & ring_mask(l))) * d) : 0.f;
        rgs[l] = ok ? Elem<T>::load(rgb + (src * a.L + l) * a.H) : 0.f;
        ig[l] = igb[(int64_t)l * a.H];
        fg[l] = fgb[(int64_t)l * a.H];
      }
    }
    float V = Elem<T>::load((const T*)a.V0 + (int64_t)b * d + (int64_t)h * a.hd + e);
    Elem<T>::store(ring + (t & 1) * d, V);
#pragma unroll
    for (int l = 0; l < kMaxL; ++l) {
      if (l < a.L) {
        V = fg[l] * V + ig[l] * rgs[l] * vs[l];
        if (l + 1 < a.L) Elem<T>::store(ring + (ring_offset(l + 1) + (t & ring_mask(l + 1))) * d, V);
      }
    }
    Elem<T>::store((T*)a.Y + (int64_t)b * d + (int64_t)h * a.hd + e, V);
  }
}

// 16-byte chunks of a row: 8 bf16 or 4 fp32 values, kept packed until used
template <typename T> struct Chunk;
template <> struct Chunk<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const uint4& v, float (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = __uint_as_float(w[j] << 16);
      o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
};
template <> struct Chunk<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const uint4& v, float (&o)[4]) {
    o[0] = __uint_as_float(v.x);
    o[1] = __uint_as_float(v.y);
    o[2] = __uint_as_float(v.z);
    o[3] = __uint_as_float(v.w);
  }
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// gate weights, streamed once per step: non-temporal loads (they leave the ring slots and history
// rows this step reads back in L2)
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldw16(const void* p) {
  const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Raw element bits, so a load's consumer (the conversion) can sit after every load is issued.
template <typename T> struct Raw;
template <> struct Raw<bf16_t> {
  __device__ __forceinline__ static uint32_t load(const bf16_t* p) { return *p; }
  __device__ __forceinline__ static float f(uint32_t r) { return __uint_as_float(r << 16); }
};
template <> struct Raw<float> {
  __device__ __forceinline__ static uint32_t load(const float* p) { return __float_as_uint(*p); }
  __device__ __forceinline__ static float f(uint32_t r) { return __uint_as_float(r); }
};

// Memory round trips are the cost of this latency-bound kernel, so loads are issued in exactly two
// waves before any barrier: (1) the position t together with everything that does not depend on
// it (gate weights, destination features A, V0, biases); (2) everything addressed through t
// (source rows of B_hist, ring slots, transmit gates). Loads are unconditional, at addresses
// clamped to a valid element, with the predicate applied to the value afterwards, or sit under a
// wave-uniform branch whose values are used only after the last request of that wave: a load
// under a branch whose value is consumed (or converted) inside the branch makes the compiler wait
// for it, and for every load before it, on the spot, serialising the round trips.
// Gate phase: wave l owns level l (L <= 16 waves); its lanes cover K in 16-byte chunks (C per
// lane), so each (row, gate) dot product ends in one DPP wave reduction and one plain LDS store.
// RPB = batch rows per workgroup, C = chunks per lane; both compile-time so the operands stay in
// registers.
template <typename T, int RPB, int C, int LMAX>
__global__ __launch_bounds__(kFusedThreads) void decode_mixer_step_kernel(StepArgs a) {
  constexpr int V = Chunk<T>::N;
  const int h = blockIdx.x;
  const int b0 = blockIdx.y * RPB;
  const int nb = min(RPB, a.B - b0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = a.L, H = a.H, hd = a.hd, GH = a.GH;   // host: L <= LMAX
  const int64_t d = (int64_t)H * hd;
  const int nchunk = GH / V;                   // host: nchunk <= 64 * C
  const int gl = min(wave, L - 1);             // gate role: wave gl owns level gl (waves < L)
  const bool gate_wave = wave < L;             // wave-uniform
  __shared__ float acc[RPB][LMAX][3];
  __shared__ float gate_i[RPB][LMAX];
  __shared__ float gate_f[RPB][LMAX];
  __shared__ float src_v[RPB][LMAX][kMaxHd];   // ring_l[slot(l, t - 2^l)] per (row, level, element)
  __shared__ float src_r[RPB][LMAX];           // rg_hist[t - 2^l, l, h] per (row, level)

  // ---- load wave 1: t and the position-independent operands
  const int64_t t = load_uniform(a.t_dev);
  uint4 w[3][C];
  uint4 av[RPB][C];
  const int64_t wrow = ((int64_t)gl * H + h) * GH;
  if (gate_wave) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t k = (int64_t)min(lane + 64 * c, nchunk - 1) * V;
      w[0][c] = ldw16((const T*)a.Wi + wrow + k);
      w[1][c] = ldw16((const T*)a.Wf + wrow + k);
      w[2][c] = ldw16((const T*)a.Wr + wrow + k);
#pragma unroll
      for (int r = 0; r < RPB; ++r) av[r][c] = ld16((const T*)a.A + (int64_t)(b0 + min(r, nb - 1)) * GH + k);
    }
  }
  const int sr = tid / hd, se = tid % hd;      // recurrence role: (row, element)
  const bool scan_role = sr < nb;
  const int64_t brow = b0 + (scan_role ? sr : 0);
  const int ar = tid / L, al = tid % L;        // activation role: (row, level)
  const bool act_role = tid < nb * L;
  // every thread reads these (their addresses are valid for any tid): under a role branch the
  // compiler converts the value inside the branch and so waits there for it, and for the weights
  // requested before it, ahead of the position-dependent requests below
  const uint32_t v0raw = Raw<T>::load((const T*)a.V0 + brow * d + (int64_t)h * hd + se);
  const int64_t gi = (int64_t)al * H + h;
  const uint32_t bir = Raw<T>::load((const T*)a.bi + gi);
  const uint32_t bfr = Raw<T>::load((const T*)a.bf + gi);
  const uint32_t brr = Raw<T>::load((const T*)a.br + gi);
  if (t < 0 || t >= a.Tmax) return;             // uniform: every thread read the same t

  // ---- load wave 2: operands addressed through t
  const int64_t gsrc = t - ((int64_t)1 << gl);
  const int64_t gsc = gsrc < 0 ? 0 : gsrc;
  uint4 bv[RPB][C];
  if (gate_wave) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t k = (int64_t)min(lane + 64 * c, nchunk - 1) * V;
#pragma unroll
      for (int r = 0; r < RPB; ++r)
        bv[r][c] = ld16((const T*)a.B_hist + ((int64_t)(b0 + min(r, nb - 1)) * a.Tmax + gsc) * GH + k);
    }
  }
  T* ring = (T*)a.V_ring + brow * a.S * d + (int64_t)h * hd + se;
  // the recurrence's sources (ring value and transmit gate of position t - 2^l per level), read
  // and staged in LDS by the waves without a gate role when there are enough of them: the loader
  // waits for its loads on the spot, which then holds up no gate readout
  {
    const int ld0 = (kFusedThreads / 64 - L) * 64 >= nb * hd ? 64 * L : 0;   // uniform
    const int u = tid - ld0;
    if (u >= 0 && u < nb * hd) {
      const int ur = u / hd, ue = u % hd;
      const int64_t urow = b0 + ur;
      const T* uring = (const T*)a.V_ring + urow * a.S * d + (int64_t)h * hd + ue;
      uint32_t vraw[LMAX], rraw[LMAX];
#pragma unroll
      for (int l = 0; l < LMAX; ++l) {          // straight-line: levels past L re-read level L-1
        const int lc = min(l, L - 1);
        const int64_t sc = max(t - ((int64_t)1 << lc), (int64_t)0);
        vraw[l] = Raw<T>::load(uring + (ring_offset(lc) + (sc & ring_mask(lc))) * d);
        rraw[l] = Raw<T>::load((const T*)a.rg_hist + ((urow * a.Tmax + sc) * L + lc) * H + h);
      }
#pragma unroll
      for (int l = 0; l < LMAX; ++l) {
        if (l < L) {
          const bool live = (t - ((int64_t)1 << l)) >= 0;
          src_v[ur][l][ue] = live ? Raw<T>::f(vraw[l]) : 0.f;
          // every lane of the row writes the same value (a predicate on this store lets the
          // compiler sink the load under it: one more round trip)
          src_r[ur][l] = live ? Raw<T>::f(rraw[l]) : 0.f;
        }
      }
    }
  }

  // ---- gate readouts of level gl: per-lane partial dots, one wave reduction per (row, gate)
  if (gate_wave) {
    const bool ok = gsrc >= 0;
#pragma unroll
    for (int r = 0; r < RPB; ++r) {
      float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        float wi[V], wf[V], wr[V], x1[V], x2[V];
        Chunk<T>::unpack(w[0][c], wi);
        Chunk<T>::unpack(w[1][c], wf);
        Chunk<T>::unpack(w[2][c], wr);
        Chunk<T>::unpack(av[r][c], x1);
        Chunk<T>::unpack(bv[r][c], x2);
        const float live = (lane + 64 * c) < nchunk ? 1.f : 0.f;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          float x = fmaxf(x1[e] + (ok ? x2[e] : 0.f), 0.f);
          x = x * x * live;
          s0 += wi[e] * x;
          s1 += wf[e] * x;
          s2 += wr[e] * x;
        }
      }
      s0 = wave_sum(s0);
      s1 = wave_sum(s1);
      s2 = wave_sum(s2);
      if (lane == 0 && r < nb) {
        acc[r][gl][0] = s0;
        acc[r][gl][1] = s1;
        acc[r][gl][2] = s2;
      }
    }
  }
  __syncthreads();                                // acc complete; every load above has landed

  // ---- sigmoid heads, masks, transmit gate of position t
  if (act_role) {
    const float okf = (t - ((int64_t)1 << al)) >= 0 ? 1.f : 0.f;
    gate_i[ar][al] = dh_sigmoid(acc[ar][al][0] + Raw<T>::f(bir)) * okf;
    gate_f[ar][al] = dh_sigmoid(acc[ar][al][1] + Raw<T>::f(bfr)) * okf + (1.f - okf);
    const float rg = dh_sigmoid(acc[ar][al][2] + Raw<T>::f(brr));
    Elem<T>::store((T*)a.rg_hist + (((int64_t)(b0 + ar) * a.Tmax + t) * L + al) * H + h, rg);
  }
  __syncthreads();

  // ---- the level recurrence over the ring buffers
  if (scan_role) {
    float v = Raw<T>::f(v0raw);
    Elem<T>::store(ring + (t & 1) * d, v);
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      if (l < L) {
        v = gate_f[sr][l] * v + gate_i[sr][l] * src_r[sr][l] * src_v[sr][l][se];
        if (l + 1 < L) Elem<T>::store(ring + (ring_offset(l + 1) + (t & ring_mask(l + 1))) * d, v);
      }
    }
    Elem<T>::store((T*)a.Y + (int64_t)(b0 + sr) * d + (int64_t)h * hd + se, v);
  }
}

// ---------------------------------------------------------------------------------------------
// Two-launch form for the graphed decoder: the gate readouts spread over one wave per
// (level, head, group of RB rows) -- the gate weights stream through ~H*L compute units instead of
// H -- and a small recurrence launch per (head, row). The first launch also gathers everything
// the recurrence reads at position-dependent addresses (the level-l ring value and transmit gate
// of position t - 2^l) into a staging buffer, so the second reads only fixed addresses.
// Staging buffer (caller-provided device memory of at least B*H*L*(4 + hd) floats), two regions:
//   coef[(b*H + h)*L + l]            = {fg, ig * r_src}     float2, from byte 0
//   vsrc[((b*H + h)*L + l)*hd + e]   = V_src[e]             model dtype, from byte vsrc_offset(B, H, L)
// with ig/fg the admit/forget gates of level l at t and r_src, V_src the level-l transmit gate and
// ring value of position t - 2^l (zeros before the sequence start). The recurrence is then
// V <- fg * V + (ig * r_src) * V_src: the same products as decode_mixer_step_kernel.
// ---------------------------------------------------------------------------------------------
__host__ __device__ __forceinline__ int64_t vsrc_offset(int B, int H, int L) {
  return (((int64_t)B * H * L * 8) + 15) & ~(int64_t)15;
}

template <typename T, int C, int RB>
__global__ __launch_bounds__(64) void decode_gates_kernel(StepArgs a, float* stage) {
  constexpr int V = Chunk<T>::N;
  const int lane = threadIdx.x;
  const int H = a.H, L = a.L, GH = a.GH, hd = a.hd;
  const int h = blockIdx.x % H, l = blockIdx.x / H;
  const int b0 = blockIdx.y * RB;
  const int nchunk = GH / V;
  const int64_t d = (int64_t)H * hd;
  float2* coef = reinterpret_cast<float2*>(stage);
  T* vsrc = reinterpret_cast<T*>(reinterpret_cast<char*>(stage) + vsrc_offset(a.B, H, L));

  // ---- t (a scalar load, so the position-dependent requests below go out as soon as it arrives,
  // while the weights are in flight), then the position-independent operands in one burst
  const int64_t t = load_uniform(a.t_dev);
  DH_ISSUE_FENCE();
  const int64_t wrow = ((int64_t)l * H + h) * GH;
  uint4 w[3][C], av[RB][C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t k = (int64_t)min(lane + 64 * c, nchunk - 1) * V;
    w[0][c] = ldw16((const T*)a.Wi + wrow + k);
    w[1][c] = ldw16((const T*)a.Wf + wrow + k);
    w[2][c] = ldw16((const T*)a.Wr + wrow + k);
#pragma unroll
    for (int r = 0; r < RB; ++r) av[r][c] = ld16((const T*)a.A + (int64_t)min(b0 + r, a.B - 1) * GH + k);
  }
  const int64_t gi = (int64_t)l * H + h;
  const uint32_t bir = Raw<T>::load((const T*)a.bi + gi);
  const uint32_t bfr = Raw<T>::load((const T*)a.bf + gi);
  const uint32_t brr = Raw<T>::load((const T*)a.br + gi);
  DH_ISSUE_FENCE();
  // out-of-range t: addresses clamped, nothing stored (no early exit: a branch before the loads
  // would make every request wait for t)
  const bool live = t >= 0 && t < a.Tmax;             // uniform

  // ---- operands addressed through t: source row of B_hist, ring value and transmit gate
  const int64_t src = t - ((int64_t)1 << l);
  const bool ok = src >= 0;
  const int64_t sc = ok && live ? src : 0;
  uint4 bv[RB][C];
  uint32_t vraw[RB][2], rraw[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int64_t b = min(b0 + r, a.B - 1);
#pragma unroll
    for (int c = 0; c < C; ++c)
      bv[r][c] = ld16((const T*)a.B_hist + (b * a.Tmax + sc) * GH + (int64_t)min(lane + 64 * c, nchunk - 1) * V);
    const T* ring = (const T*)a.V_ring + (b * a.S + ring_offset(l) + (sc & ring_mask(l))) * d + (int64_t)h * hd;
#pragma unroll
    for (int q = 0; q < 2; ++q) vraw[r][q] = Raw<T>::load(ring + min(lane + 64 * q, hd - 1));
    rraw[r] = Raw<T>::load((const T*)a.rg_hist + ((b * a.Tmax + sc) * L + l) * H + h);
  }
  DH_ISSUE_FENCE();

  // ---- the three dot products of each row, gates, staging
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      float wi[V], wf[V], wr[V], x1[V], x2[V];
      Chunk<T>::unpack(w[0][c], wi);
      Chunk<T>::unpack(w[1][c], wf);
      Chunk<T>::unpack(w[2][c], wr);
      Chunk<T>::unpack(av[r][c], x1);
      Chunk<T>::unpack(bv[r][c], x2);
      const float live = (lane + 64 * c) < nchunk ? 1.f : 0.f;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float x = fmaxf(x1[e] + (ok ? x2[e] : 0.f), 0.f);
        x = x * x * live;
        s0 += wi[e] * x;
        s1 += wf[e] * x;
        s2 += wr[e] * x;
      }
    }
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const int b = b0 + r;
    if (b < a.B && live) {                             // uniform
      const int64_t rec = ((int64_t)b * H + h) * L + l;
      if (lane == 0) {
        const float okf = ok ? 1.f : 0.f;
        const float ig = dh_sigmoid(s0 + Raw<T>::f(bir)) * okf;
        const float fg = dh_sigmoid(s1 + Raw<T>::f(bfr)) * okf + (1.f - okf);
        const float rs = ok ? Raw<T>::f(rraw[r]) : 0.f;
        coef[rec] = make_float2(fg, ig * rs);
        Elem<T>::store((T*)a.rg_hist + (((int64_t)b * a.Tmax + t) * L + l) * H + h, dh_sigmoid(s2 + Raw<T>::f(brr)));
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int e = lane + 64 * q;
        if (e < hd) {                                  // the ring value's own bits (exact)
          const uint32_t bits = ok ? vraw[r][q] : 0u;
          if constexpr (sizeof(T) == 2)
            vsrc[rec * hd + e] = (T)bits;
          else
            vsrc[rec * hd + e] = __uint_as_float(bits);
        }
      }
    }
  }
}

// The level recurrence of one (head, row) from the staged gates and sources: one thread per element.
template <typename T, int LMAX>
__global__ __launch_bounds__(kMaxHd) void decode_scan_kernel(StepArgs a, const float* stage) {
  const int h = blockIdx.x, b = blockIdx.y, e = threadIdx.x;
  const int H = a.H, L = a.L, hd = a.hd;
  const int64_t d = (int64_t)H * hd;
  const int64_t t = load_uniform(a.t_dev);             // requested first, waited for last
  DH_ISSUE_FENCE();
  const float2* coef = reinterpret_cast<const float2*>(stage) + ((int64_t)b * H + h) * L;
  const T* vsrc = reinterpret_cast<const T*>(reinterpret_cast<const char*>(stage) + vsrc_offset(a.B, H, L)) +
                  ((int64_t)b * H + h) * L * hd + e;
  float2 cf[LMAX];
  uint32_t vr[LMAX];
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {                     // levels past L re-read level L-1 (unused)
    const int lc = min(l, L - 1);
    cf[l] = coef[lc];
    vr[l] = Raw<T>::load(vsrc + (int64_t)lc * hd);
  }
  const uint32_t v0raw = Raw<T>::load((const T*)a.V0 + (int64_t)b * d + (int64_t)h * hd + e);
  DH_ISSUE_FENCE();
  // out-of-range t: nothing stored (no early exit: a branch here lets the compiler move the staged
  // loads behind the wait for t)
  const bool live = t >= 0 && t < a.Tmax;             // uniform
  T* ring = (T*)a.V_ring + (int64_t)b * a.S * d + (int64_t)h * hd + e;
  float v = Raw<T>::f(v0raw);
  if (live) Elem<T>::store(ring + (t & 1) * d, v);
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    if (l < L) {
      v = cf[l].x * v + cf[l].y * Raw<T>::f(vr[l]);
      if (live && l + 1 < L) Elem<T>::store(ring + (ring_offset(l + 1) + (t & ring_mask(l + 1))) * d, v);
    }
  }
  if (live) Elem<T>::store((T*)a.Y + (int64_t)b * d + (int64_t)h * hd + e, v);
}

template <typename T, int RPB, int C, int LMAX>
void launch_fused(const StepArgs& a, hipStream_t s) {
  dim3 grid(a.H, (a.B + RPB - 1) / RPB), block(kFusedThreads);
  decode_mixer_step_kernel<T, RPB, C, LMAX><<<grid, block, 0, s>>>(a);
}

template <typename T, int LMAX>
void dispatch_rc(const StepArgs& a, int rpb, int C, hipStream_t s) {
  if (C <= 1) {
    if (rpb == 1) launch_fused<T, 1, 1, LMAX>(a, s); else launch_fused<T, 2, 1, LMAX>(a, s);
  } else if (C == 2) {
    if (rpb == 1) launch_fused<T, 1, 2, LMAX>(a, s); else launch_fused<T, 2, 2, LMAX>(a, s);
  } else {
    launch_fused<T, 1, 4, LMAX>(a, s);
  }
}

template <typename T>
void dispatch_fused(const StepArgs& a, int rpb, int C, hipStream_t s) {
  if (a.L <= 8) dispatch_rc<T, 8>(a, rpb, C, s);
  else if (a.L <= 12) dispatch_rc<T, 12>(a, rpb, C, s);
  else dispatch_rc<T, 16>(a, rpb, C, s);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void step_gates_kernel(StepArgs a) {
  const int64_t t = load_uniform(a.t_dev);
  if (t < 0 || t >= a.Tmax) return;
  int h, l;
  block_coords(blockIdx.x, a.H, a.L, h, l);
  gates_phase<T>(a, h, l, t);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void step_scan_kernel(StepArgs a) {
  const int64_t t = load_uniform(a.t_dev);
  if (t < 0 || t >= a.Tmax) return;
  scan_phase<T>(a, blockIdx.x, t);
}


bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

int check_common(const char* who, int dtype, int B, int Tmax, int GH, int H, int hd, int L) {
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && Tmax >= 1, DH_ERR_INVALID_ARG, "%s: B=%d Tmax=%d must be >= 1", who, B, Tmax);
  DH_REQUIRE(L >= 1 && L <= kMaxL, DH_ERR_UNSUPPORTED_SHAPE, "%s: L=%d not in [1,%d]", who, L, kMaxL);
  DH_REQUIRE(H >= 1 && H <= 64, DH_ERR_UNSUPPORTED_SHAPE, "%s: H=%d not in [1,64]", who, H);
  DH_REQUIRE(hd == 16 || hd == 32 || hd == 64 || hd == 128, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: hd=%d not in {16,32,64,128}", who, hd);
  DH_REQUIRE(GH >= 64 && GH % 64 == 0, DH_ERR_UNSUPPORTED_SHAPE, "%s: GH=%d not a multiple of 64", who, GH);
  return DH_OK;
}

// ---------------------------------------------------------------------------------------------
// dh_decode_scan_out (batch 1): the recurrence of dh_decode_scan fused into the out-projection
// GEMV that consumes its Y (linear_out + residual, reference decoding.py:473-476), saving a launch
// per tree layer. The out-projection needs all of Y in every workgroup, so every workgroup runs the
// whole recurrence (d elements, 4 per thread) from the staging record -- copied cooperatively into
// LDS with 16-byte loads (26 KB at the released shape, L2-resident) -- and workgroup 0 alone writes
// the ring slots of position t and Y. Order of requests: t (scalar), the staging record and V0,
// the residual, then the wave's weight row; the LDS copy then waits for the staging loads only
// (loads return in issue order), Y goes to LDS in the model dtype (rounded where the two-launch path
// stores it), and each wave's output row is a dot product with DPP reductions, as in dh_decode_gemv.
// Out-of-range t: nothing is written.
// ---------------------------------------------------------------------------------------------
// four consecutive elements as one 8-byte (bf16) or 16-byte (fp32) access
template <typename T> struct Quad;
template <> struct Quad<bf16_t> {
  __device__ __forceinline__ static void load(const bf16_t* p, float (&o)[4]) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    o[0] = __uint_as_float(w.x << 16);
    o[1] = __uint_as_float(w.x & 0xffff0000u);
    o[2] = __uint_as_float(w.y << 16);
    o[3] = __uint_as_float(w.y & 0xffff0000u);
  }
  __device__ __forceinline__ static void store(bf16_t* p, const float (&v)[4]) {
    *reinterpret_cast<uint2*>(p) = make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                                              (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
  }
};
template <> struct Quad<float> {
  __device__ __forceinline__ static void load(const float* p, float (&o)[4]) {
    const float4 w = *reinterpret_cast<const float4*>(p);
    o[0] = w.x;
    o[1] = w.y;
    o[2] = w.z;
    o[3] = w.w;
  }
  __device__ __forceinline__ static void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

struct ScanOutArgs {
  const void* V0;
  const float* stage;
  const int64_t* t_dev;
  void* V_ring;
  void* Y;
  const void* W;              // (N, d) linear_out weight, row-major
  const void* resid;          // residual row (model dtype)
  const int64_t* resid_rows;  // nullable: the residual row is resid + resid_rows[0] * resid_stride
  int64_t resid_stride;
  void* out;                  // (N) output row; may alias the residual row
  int Tmax, S, H, hd, L, N;
};
constexpr int kSOThreads = 256;
#ifndef DH_SCANOUT_ROWS
#define DH_SCANOUT_ROWS 1
#endif
constexpr int kSORows = DH_SCANOUT_ROWS;   // output rows per wave (each workgroup redoes the recurrence)
constexpr int kSOEpt = 4;                  // recurrence elements per thread: d <= 1024

template <typename T, int CG, int LMAX, int RW>
__global__ __launch_bounds__(kSOThreads) void decode_scan_out_kernel(ScanOutArgs a) {
  constexpr int kMaxD = kSOEpt * kSOThreads;           // 1024
  constexpr int VCH = kMaxD * LMAX * (int)sizeof(T) / 16 / kSOThreads;   // staged 16-byte chunks per thread
  __shared__ uint4 svs[kMaxD * LMAX * sizeof(T) / 16];  // ring sources of batch row 0, (h, l, e)
  __shared__ float2 scf[64 * LMAX];                      // {fg, ig * r_src} of row 0, (h, l)
  __shared__ uint4 sy[CG * 64];                          // Y in the model dtype
  constexpr int V = Chunk<T>::N;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, L = a.L, hd = a.hd;
  const int d = H * hd;
  const int nchunk = d / V;
  const int64_t t = load_uniform(a.t_dev);
  DH_ISSUE_FENCE();

  // ---- batch row 0's staging record (H*L coefficient pairs, H*L*hd sources) and V0, all at fixed
  // addresses written by the gates launch: one cooperative copy into LDS, 16-byte loads
  const int ncf = H * L;
  const int nvs = ncf * hd * (int)sizeof(T) / 16;
  const float2* gcf = reinterpret_cast<const float2*>(a.stage);
  const uint4* gvs = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(a.stage) + vsrc_offset(1, H, L));
  // (four word arrays: an array of uint4 here is kept in private memory by the compiler)
  uint32_t cvx[VCH], cvy[VCH], cvz[VCH], cvw[VCH];
#pragma unroll
  for (int j = 0; j < VCH; ++j) {
    const uint4 q = gvs[min(tid + j * kSOThreads, nvs - 1)];
    cvx[j] = q.x; cvy[j] = q.y; cvz[j] = q.z; cvw[j] = q.w;
  }
  float2 cc[(64 * LMAX + kSOThreads - 1) / kSOThreads];
#pragma unroll
  for (int j = 0; j < (64 * LMAX + kSOThreads - 1) / kSOThreads; ++j) cc[j] = gcf[min(tid + j * kSOThreads, ncf - 1)];
  const int e0 = min(tid * kSOEpt, d - kSOEpt);
  uint32_t v0r[kSOEpt];
#pragma unroll
  for (int q = 0; q < kSOEpt; ++q) v0r[q] = Raw<T>::load((const T*)a.V0 + e0 + q);
  // the residual of output row nbase + lane % RW (lane r < RW uses it)
  const int nbase = ((int)blockIdx.x * (kSOThreads / 64) + wave) * RW;
  const int64_t rrow = a.resid_rows ? load_uniform(a.resid_rows) : 0;
  const uint32_t rc = Raw<T>::load((const T*)a.resid + rrow * a.resid_stride + min(nbase + lane % RW, a.N - 1));
  DH_ISSUE_FENCE();

  // ---- the wave's RW weight rows, one burst
  uint4 w[RW][CG];
#pragma unroll
  for (int c = 0; c < CG; ++c)
#pragma unroll
    for (int r = 0; r < RW; ++r)
      w[r][c] = ld16((const T*)a.W + (int64_t)min(nbase + r, a.N - 1) * d + (int64_t)min(lane + 64 * c, nchunk - 1) * V);
  DH_ISSUE_FENCE();

  // ---- stage into LDS (waits for the staging loads only; clamped duplicates rewrite the last slot)
#pragma unroll
  for (int j = 0; j < VCH; ++j) svs[min(tid + j * kSOThreads, nvs - 1)] = make_uint4(cvx[j], cvy[j], cvz[j], cvw[j]);
#pragma unroll
  for (int j = 0; j < (64 * LMAX + kSOThreads - 1) / kSOThreads; ++j) scf[min(tid + j * kSOThreads, ncf - 1)] = cc[j];
  __syncthreads();

  // ---- this thread's operands of every level, then the recurrence of elements e0 .. e0+3 (one
  // head), branch-free; workgroup 0 then writes the ring slots and Y
  const bool live = t >= 0 && t < a.Tmax;
  const bool writer = live && blockIdx.x == 0 && tid * kSOEpt < d;
  const int h = e0 / hd, eh = e0 - h * hd;
  const T* lvs = reinterpret_cast<const T*>(svs);
  float2 cf[LMAX];
  float vs[LMAX][kSOEpt];
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    const int lc = min(l, L - 1);
    cf[l] = scf[h * L + lc];
    Quad<T>::load(lvs + (int64_t)(h * L + lc) * hd + eh, vs[l]);
  }
  float v[kSOEpt];
#pragma unroll
  for (int q = 0; q < kSOEpt; ++q) v[q] = Raw<T>::f(v0r[q]);
  float hist[LMAX][kSOEpt];                              // state entering level l + 1
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    const bool on = l < L;                               // uniform
#pragma unroll
    for (int q = 0; q < kSOEpt; ++q) {
      // one explicit fused multiply-add (the one-launch step evaluates the same form)
      const float nv = __builtin_fmaf(cf[l].y, vs[l][q], cf[l].x * v[q]);
      v[q] = on ? nv : v[q];
      hist[l][q] = v[q];
    }
  }
  if (writer) {
    T* ring = (T*)a.V_ring + e0;
    float v0f[kSOEpt];
#pragma unroll
    for (int q = 0; q < kSOEpt; ++q) v0f[q] = Raw<T>::f(v0r[q]);
    Quad<T>::store(ring + (t & 1) * d, v0f);
#pragma unroll
    for (int l = 0; l + 1 < LMAX; ++l)
      if (l + 1 < L) Quad<T>::store(ring + (ring_offset(l + 1) + (t & ring_mask(l + 1))) * d, hist[l]);
    Quad<T>::store((T*)a.Y + e0, v);
  }
  if (tid * kSOEpt < d) Quad<T>::store(reinterpret_cast<T*>(sy) + e0, v);
  __syncthreads();

  // ---- out[n] = round(round(W[n] . Y) + resid[n]) for the wave's rows
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) acc[r] = 0.f;
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int ch = lane + 64 * c;
    float yv[V];
    if constexpr (sizeof(T) != 2) Chunk<T>::unpack(sy[min(ch, nchunk - 1)], yv);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float part = 0.f;
      if constexpr (sizeof(T) == 2) {
        part = dot8_bf16(w[r][c], sy[min(ch, nchunk - 1)]);   // as the one-launch step's dot_rows
      } else {
        float wv[V];
        Chunk<T>::unpack(w[r][c], wv);
#pragma unroll
        for (int e = 0; e < V; ++e) part += wv[e] * yv[e];
      }
      acc[r] += ch < nchunk ? part : 0.f;
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) acc[r] = wave_sum(acc[r]);
  if (lane < RW && live && nbase + lane < a.N) {
    float v0 = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) v0 = r == lane ? acc[r] : v0;
    uint32_t rv = rc;
    asm volatile("" : "+v"(rv));                        // converted here, not beside its load
    Elem<T>::store((T*)a.out + nbase + lane, Elem<T>::round(Elem<T>::round(v0) + Raw<T>::f(rv)));
  }
}

}  // namespace

extern "C" int dh_decode_mixer_step(int dtype, const void* A, const void* B_hist, const void* Wi,
                                    const void* Wf, const void* Wr, const void* bi, const void* bf,
                                    const void* br, const int64_t* t_dev, void* rg_hist,
                                    void* V_ring, const void* V0, void* Y, int B, int Tmax, int S, int GH,
                                    int H, int hd, int L, void* stream) {
  const char* who = "dh_decode_mixer_step";
  int st = check_common(who, dtype, B, Tmax, GH, H, hd, L);
  if (st) return st;
  DH_REQUIRE(S == (int)ring_offset(L), DH_ERR_INVALID_ARG, "%s: S=%d but L=%d needs %lld ring slots", who, S, L,
             (long long)ring_offset(L));
  DH_REQUIRE(A && B_hist && Wi && Wf && Wr && bi && bf && br && t_dev && rg_hist && V_ring && V0 && Y,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(aligned(A, 16) && aligned(B_hist, 16) && aligned(Wi, 16) && aligned(Wf, 16) && aligned(Wr, 16),
             DH_ERR_INVALID_ARG, "%s: A/B_hist/W need 16-byte alignment", who);
  const int vec = dtype == DH_BF16 ? 8 : 4;
  const int C = (GH / vec + 63) / 64;          // 16-byte chunks per lane of one weight row
  DH_REQUIRE(C <= 4, DH_ERR_UNSUPPORTED_SHAPE, "%s: GH=%d exceeds %d elements per gate row", who, GH, 4 * 64 * vec);
  // two rows per workgroup (sharing the gate weights) while one row per workgroup would leave fewer
  // than 128 workgroups and two rows' operands still fit the register budget; from 128 (head, row)
  // pairs on, one row each (batch 16 x 16 heads: 0.708 vs 0.722 ms per decode step)
  const int rpb = (B >= 2 && B * H < 128 && C <= 2 && 2 * hd <= kFusedThreads) ? 2 : 1;
  StepArgs a{A, B_hist, Wi, Wf, Wr, bi, bf, br, t_dev, rg_hist, V_ring, V0, Y, nullptr, nullptr,
             B, Tmax, S, GH, H, hd, L, rpb};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32)
    dispatch_fused<float>(a, rpb, C, s);
  else
    dispatch_fused<bf16_t>(a, rpb, C, s);
  return dh_check_launch(who);
}

template <typename T, int C>
void launch_gates(const StepArgs& a, float* stage, hipStream_t s) {
  if (a.B >= 4) {
    dim3 grid(a.H * a.L, (a.B + 3) / 4);
    decode_gates_kernel<T, C, 4><<<grid, dim3(64), 0, s>>>(a, stage);
  } else {
    dim3 grid(a.H * a.L, a.B);
    decode_gates_kernel<T, C, 1><<<grid, dim3(64), 0, s>>>(a, stage);
  }
}

template <typename T>
void launch_scan(const StepArgs& a, const float* stage, hipStream_t s) {
  dim3 grid(a.H, a.B), block(a.hd);
  if (a.L <= 8) decode_scan_kernel<T, 8><<<grid, block, 0, s>>>(a, stage);
  else if (a.L <= 12) decode_scan_kernel<T, 12><<<grid, block, 0, s>>>(a, stage);
  else decode_scan_kernel<T, 16><<<grid, block, 0, s>>>(a, stage);
}

extern "C" int dh_decode_gates(int dtype, const void* A, const void* B_hist, const void* Wi, const void* Wf,
                               const void* Wr, const void* bi, const void* bf, const void* br, const int64_t* t_dev,
                               void* rg_hist, const void* V_ring, float* stage, int B, int Tmax, int S, int GH,
                               int H, int hd, int L, void* stream) {
  const char* who = "dh_decode_gates";
  int st = check_common(who, dtype, B, Tmax, GH, H, hd, L);
  if (st) return st;
  DH_REQUIRE(S == (int)ring_offset(L), DH_ERR_INVALID_ARG, "%s: S=%d but L=%d needs %lld ring slots", who, S, L,
             (long long)ring_offset(L));
  DH_REQUIRE(A && B_hist && Wi && Wf && Wr && bi && bf && br && t_dev && rg_hist && V_ring && stage,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(aligned(A, 16) && aligned(B_hist, 16) && aligned(Wi, 16) && aligned(Wf, 16) && aligned(Wr, 16),
             DH_ERR_INVALID_ARG, "%s: A/B_hist/W need 16-byte alignment", who);
  const int vec = dtype == DH_BF16 ? 8 : 4;
  const int C = (GH / vec + 63) / 64;
  DH_REQUIRE(C <= 4, DH_ERR_UNSUPPORTED_SHAPE, "%s: GH=%d exceeds %d elements per gate row", who, GH, 4 * 64 * vec);
  StepArgs a{A, B_hist, Wi, Wf, Wr, bi, bf, br, t_dev, rg_hist, (void*)V_ring, nullptr, nullptr, nullptr, nullptr,
             B, Tmax, S, GH, H, hd, L, 0};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32) {
    if (C <= 1) launch_gates<float, 1>(a, stage, s);
    else if (C == 2) launch_gates<float, 2>(a, stage, s);
    else launch_gates<float, 4>(a, stage, s);
  } else {
    if (C <= 1) launch_gates<bf16_t, 1>(a, stage, s);
    else if (C == 2) launch_gates<bf16_t, 2>(a, stage, s);
    else launch_gates<bf16_t, 4>(a, stage, s);
  }
  return dh_check_launch(who);
}

extern "C" int dh_decode_scan(int dtype, const void* V0, const float* stage, const int64_t* t_dev, void* V_ring,
                              void* Y, int B, int Tmax, int S, int H, int hd, int L, void* stream) {
  const char* who = "dh_decode_scan";
  int st = check_common(who, dtype, B, Tmax, 64, H, hd, L);
  if (st) return st;
  DH_REQUIRE(S == (int)ring_offset(L), DH_ERR_INVALID_ARG, "%s: S=%d but L=%d needs %lld ring slots", who, S, L,
             (long long)ring_offset(L));
  DH_REQUIRE(V0 && stage && t_dev && V_ring && Y, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  StepArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, t_dev, nullptr, V_ring, V0, Y,
             nullptr, nullptr, B, Tmax, S, 64, H, hd, L, 0};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32)
    launch_scan<float>(a, stage, s);
  else
    launch_scan<bf16_t>(a, stage, s);
  return dh_check_launch(who);
}

extern "C" int dh_step_gates(int dtype, const void* A, const void* B_hist, const void* Wi, const void* Wf,
                             const void* Wr, const void* bi, const void* bf, const void* br,
                             const int64_t* t_dev, float* IG, float* FG, void* rg_hist, int B, int Tmax,
                             int GH, int H, int L, void* stream) {
  const char* who = "dh_step_gates";
  int st = check_common(who, dtype, B, Tmax, GH, H, 64, L);
  if (st) return st;
  DH_REQUIRE(A && B_hist && Wi && Wf && Wr && bi && bf && br && t_dev && IG && FG && rg_hist,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(aligned(A, 16) && aligned(B_hist, 16) && aligned(Wi, 16) && aligned(Wf, 16) && aligned(Wr, 16),
             DH_ERR_INVALID_ARG, "%s: A/B_hist/W need 16-byte alignment", who);
  StepArgs a{A, B_hist, Wi, Wf, Wr, bi, bf, br, t_dev, rg_hist, nullptr, nullptr, nullptr, IG, FG,
             B, Tmax, 0, GH, H, 64, L, 0};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32)
    step_gates_kernel<float><<<dim3(H * L), dim3(kThreads), 0, s>>>(a);
  else
    step_gates_kernel<bf16_t><<<dim3(H * L), dim3(kThreads), 0, s>>>(a);
  return dh_check_launch(who);
}

extern "C" int dh_step_scan(int dtype, const void* V0, const float* IG, const float* FG, const void* rg_hist,
                            void* V_ring, const int64_t* t_dev, void* Y, int B, int Tmax, int S, int H, int hd,
                            int L, void* stream) {
  const char* who = "dh_step_scan";
  int st = check_common(who, dtype, B, Tmax, 64, H, hd, L);
  if (st) return st;
  DH_REQUIRE(S == (int)ring_offset(L), DH_ERR_INVALID_ARG, "%s: S=%d but L=%d needs %lld ring slots", who, S, L,
             (long long)ring_offset(L));
  DH_REQUIRE(V0 && IG && FG && rg_hist && V_ring && t_dev && Y, DH_ERR_INVALID_ARG, "%s: null pointer argument",
             who);
  StepArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, t_dev, (void*)rg_hist,
             V_ring, V0, Y, (float*)IG, (float*)FG, B, Tmax, S, 64, H, hd, L, 0};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32)
    step_scan_kernel<float><<<dim3(H), dim3(kThreads), 0, s>>>(a);
  else
    step_scan_kernel<bf16_t><<<dim3(H), dim3(kThreads), 0, s>>>(a);
  return dh_check_launch(who);
}

extern "C" int dh_decode_scan_out(int dtype, const void* V0, const float* stage, const int64_t* t_dev,
                                  void* V_ring, void* Y, const void* W, const void* resid,
                                  const int64_t* resid_rows, int64_t resid_stride, void* out, int Tmax, int S,
                                  int H, int hd, int L, int N, void* stream) {
  const char* who = "dh_decode_scan_out";
  int st = check_common(who, dtype, 1, Tmax, 64, H, hd, L);
  if (st) return st;
  const int d = H * hd;
  const int vec = dtype == DH_BF16 ? 8 : 4;
  DH_REQUIRE(d <= kSOEpt * kSOThreads && d % vec == 0 && (d / vec + 63) / 64 <= 4, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: d=%d (H*hd) must be <= %d", who, d, kSOEpt * kSOThreads);
  DH_REQUIRE(S == (int)ring_offset(L), DH_ERR_INVALID_ARG, "%s: S=%d but L=%d needs %lld ring slots", who, S, L,
             (long long)ring_offset(L));
  DH_REQUIRE(N >= 1, DH_ERR_INVALID_ARG, "%s: N=%d", who, N);
  DH_REQUIRE(V0 && stage && t_dev && V_ring && Y && W && resid && out, DH_ERR_INVALID_ARG,
             "%s: null pointer argument", who);
  DH_REQUIRE(aligned(stage, 16) && aligned(W, 16), DH_ERR_INVALID_ARG, "%s: stage/W need 16-byte alignment", who);
  ScanOutArgs a{V0, stage, t_dev, V_ring, Y, W, resid, resid_rows, resid_stride, out, Tmax, S, H, hd, L, N};
  hipStream_t s = (hipStream_t)stream;
  const int grid = (N + (kSOThreads / 64) * kSORows - 1) / ((kSOThreads / 64) * kSORows);
  const int C = (d / vec + 63) / 64;
#define DH_SO(TT, CC, LL) decode_scan_out_kernel<TT, CC, LL, kSORows><<<dim3(grid), dim3(kSOThreads), 0, s>>>(a)
  if (dtype == DH_BF16) {
    if (L <= 8) { if (C <= 2) DH_SO(bf16_t, 2, 8); else DH_SO(bf16_t, 4, 8); }
    else if (L <= 12) { if (C <= 2) DH_SO(bf16_t, 2, 12); else DH_SO(bf16_t, 4, 12); }
    else { if (C <= 2) DH_SO(bf16_t, 2, 16); else DH_SO(bf16_t, 4, 16); }
  } else {
    if (L <= 8) { if (C <= 2) DH_SO(float, 2, 8); else DH_SO(float, 4, 8); }
    else if (L <= 12) { if (C <= 2) DH_SO(float, 2, 12); else DH_SO(float, 4, 12); }
    else { if (C <= 2) DH_SO(float, 2, 16); else DH_SO(float, 4, 16); }
  }
#undef DH_SO
  return dh_check_launch(who);
}
