// The mixer's input projections as one MFMA GEMM, for gfx950:
//   out_s[m, n] = sum_k X[m, k] * W_s[n, k]        s < nseg <= 3, W_s (N_s, K) row-major (nn.Linear)
// (reference dispatcher_hybrid/modeling_dispatcher.py:63-74: V0 = linear_in(x), A = gate_hidden(x),
// B = gate_hidden_src(x) -- three GEMMs over the same rows, done here as one launch over the
// concatenated N = N_0 + N_1 + N_2 columns). fp32 accumulation; bf16 outputs rounded once.
//
// Work decomposition: a workgroup (4 wave64s, a 2 x 2 grid) computes a square output tile of
// 32 * WT rows and columns; each wave a quadrant of WT x WT MFMA tiles of 16 x 16
// (v_mfma_f32_16x16x32_bf16; fp32 models use v_mfma_f32_16x16x4f32). Two tile sizes:
//   WT = 4: 128 x 128 tiles, for launches with too few 256 x 256 tiles to fill the 256 CUs;
//   WT = 8: 256 x 256 tiles (bf16), for many rows: each wave's 128 x 128 quadrant reads 512 LDS bytes
//           per k for 32 KFLOP, half the LDS traffic per MFMA of the 128 x 128 tile, whose 64 x 64
//           quadrants need the LDS at its full read rate to keep the MFMA pipe busy.
// K advances in tiles of 128 bytes per row (64 bf16 / 32 fp32): both operand tiles are staged in LDS
// with a 16-byte row pad (conflict-free 16-byte fragment reads), double-buffered, the next tile's
// global loads in flight in registers while the current one is multiplied; one barrier per K tile.
// The weight tile is the MFMA's A operand and the activation tile its B operand, so the accumulator
// of a lane holds four consecutive output columns of one output row: the epilogue writes 8 (bf16) or
// 16 (fp32) contiguous bytes per lane and MFMA tile.
// Block order is XCD-aware: with round-robin dispatch over the 8 XCDs, block id % 8 picks the XCD,
// and every column tile of a row tile goes to the same XCD, so the row tile's activations are
// fetched once into that XCD's L2.
#include "dh_common.h"

namespace {

constexpr int kBM = 128;                  // output rows (activation rows) per workgroup
constexpr int kBN = 128;                  // output columns (weight rows) per workgroup
constexpr int kThreads = 256;
constexpr int kRowBytes = 128;            // K bytes of a staged row
constexpr int kPad = 16;
constexpr int kRS = kRowBytes + kPad;     // LDS row stride
constexpr int kTileBytes = 128 * kRS;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct GemmArgs {
  const void* X;
  int64_t ldx;
  const void* W[3];
  void* out[3];
  int64_t ldo[3];
  int N[3];
  int nseg, M, K, Ntot;
  int mtiles, ntiles;
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// segment and local column of concatenated column n (uniform selects over the argument fields)
__device__ __forceinline__ int seg_of(const GemmArgs& a, int n, int& local) {
  const int N0 = a.N[0], N1 = a.N[1];
  const bool in1 = a.nseg > 1 && n >= N0;
  const bool in2 = a.nseg > 2 && n >= N0 + N1;
  local = n - (in2 ? N0 + N1 : (in1 ? N0 : 0));
  return in2 ? 2 : (in1 ? 1 : 0);
}
template <typename P>
__device__ __forceinline__ P pick(int s, P p0, P p1, P p2) {
  return s == 0 ? p0 : (s == 1 ? p1 : p2);
}

template <typename T> struct Frag;
template <> struct Frag<bf16_t> {
  static constexpr int VE = 8;            // elements per 16-byte chunk
  static constexpr int KSTEPS = 2;        // MFMA k-steps of 32 per staged tile
  // one 16x16x32 step: lane (r, g) holds k = 8g .. 8g+7 of the step for row / column r
  __device__ __forceinline__ static void mma(f32x4& acc, const uint4& w, const uint4& x) {
    bf16x8 a, b;
    __builtin_memcpy(&a, &w, 16);
    __builtin_memcpy(&b, &x, 16);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static void store4(bf16_t* p, const f32x4& v) {
    const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
    *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
  }
};
template <> struct Frag<float> {
  static constexpr int VE = 4;
  static constexpr int KSTEPS = 2;        // steps of 16 k: lane group g holds k = 4g .. 4g+3
  // four 16x16x4 MFMAs; MFMA j takes k = 4g + j on both operands
  __device__ __forceinline__ static void mma(f32x4& acc, const uint4& w, const uint4& x) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(w.x), __uint_as_float(x.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(w.y), __uint_as_float(x.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(w.z), __uint_as_float(x.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(w.w), __uint_as_float(x.w), acc, 0, 0, 0);
  }
  __device__ __forceinline__ static void store4(float* p, const f32x4& v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

template <typename T>
__global__ __launch_bounds__(kThreads) void proj_gemm_kernel(GemmArgs a) {
  __shared__ __align__(16) unsigned char smem[2][2][kTileBytes];   // [buffer][weights | activations]
  typedef Frag<T> F;
  constexpr int VE = F::VE;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;             // the wave's 64 x 64 quadrant

  // tile of this workgroup: XCD x = id % 8 takes row tiles x, x + 8, ..., each with all its
  // column tiles in a row
  const int id = blockIdx.x;
  const int xcd = id & 7, slot = id >> 3;
  const int mt = (slot / a.ntiles) * 8 + xcd, nt = slot % a.ntiles;
  if (mt >= a.mtiles) return;                          // uniform
  const int m0 = mt * kBM, n0 = nt * kBN;

  // global -> LDS mapping: chunk c = tid + 256 q is row c / 8, 16-byte chunk c % 8 of the row
  const T* xp[4];
  const T* wp[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = tid + kThreads * q;
    const int row = c >> 3, cc = c & 7;
    const int m = min(m0 + row, a.M - 1);
    xp[q] = (const T*)a.X + (int64_t)m * a.ldx + cc * VE;
    int loc;
    const int n = min(n0 + row, a.Ntot - 1);
    const int s = seg_of(a, n, loc);
    wp[q] = (const T*)pick(s, a.W[0], a.W[1], a.W[2]) + (int64_t)loc * a.K + cc * VE;
  }
  uint4 px[4], pw[4];
  auto fetch = [&](int kt) {
    const int k0 = kt * (kRowBytes / (int)sizeof(T));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pw[q] = ld16(wp[q] + k0);
      px[q] = ld16(xp[q] + k0);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + kThreads * q;
      const int off = (c >> 3) * kRS + (c & 7) * 16;
      *reinterpret_cast<uint4*>(&smem[buf][0][off]) = pw[q];
      *reinterpret_cast<uint4*>(&smem[buf][1][off]) = px[q];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = a.K / (kRowBytes / (int)sizeof(T));
  fetch(0);
  stage(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) fetch(kt + 1);                    // in flight during the multiply
#pragma unroll
    for (int ks = 0; ks < F::KSTEPS; ++ks) {
      uint4 wf[4], xf[4];
      const int kb = ks * 64 + g * 16;                 // byte offset of this lane's k chunk
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wf[j] = *reinterpret_cast<const uint4*>(&smem[cur][0][(wn * 64 + j * 16 + r) * kRS + kb]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xf[i] = *reinterpret_cast<const uint4*>(&smem[cur][1][(wm * 64 + i * 16 + r) * kRS + kb]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) F::mma(acc[j][i], wf[j], xf[i]);
    }
    if (kt + 1 < nk) stage(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: acc[j][i] = out[m][n .. n+3], m = m0 + wm*64 + i*16 + r, n = n0 + wn*64 + j*16 + 4g
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + j * 16 + 4 * g;
    int loc;
    const int s = seg_of(a, n, loc);
    T* o = (T*)pick(s, a.out[0], a.out[1], a.out[2]);
    const int64_t ld = pick(s, a.ldo[0], a.ldo[1], a.ldo[2]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + wm * 64 + i * 16 + r;
      if (m < a.M && n < a.Ntot) F::store4(o + (int64_t)m * ld + loc, acc[j][i]);
    }
  }
}

// LDS byte address of a __shared__ pointer (the M0 operand of global_load_lds)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int N>
__device__ __forceinline__ void wait_vm() {          // s_waitcnt vmcnt(N), other counters untouched
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Output of a bf16 tile with 16-byte stores: MFMA tiles j and j + 1 (16 columns each) of a lane's
// row are exchanged between lane rows g and g ^ 1 (v_permlane16_swap), after which lane (r, g) holds
// 8 consecutive columns: 16 j' + 16 (g & 1) + 8 (g >> 1) .. + 7 of the 32-column pair j' = 2p.
// Non-temporal: the output is not read again by the launch, so it need not displace the operand
// tiles from L2. Needs column pairs in one segment (segment widths multiples of 8) and 16-byte
// aligned output rows.
template <int TM, int TN, int WGM>
__device__ __forceinline__ void store_tile_x4(const GemmArgs& a, const f32x4 (&acc)[TN][TM], int m0, int n0, int wm,
                                              int wn, int r, int g) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  static_assert(TN % 2 == 0, "column tiles in pairs");
#pragma unroll
  for (int p = 0; p < TN / 2; ++p) {
    const int n = n0 + wn * 16 * TN + p * 32 + (g & 1) * 16 + (g >> 1) * 8;
    int loc;
    const int s = seg_of(a, min(n, a.Ntot - 1), loc);
    bf16_t* o = (bf16_t*)pick(s, a.out[0], a.out[1], a.out[2]);
    const int64_t ld = pick(s, a.ldo[0], a.ldo[1], a.ldo[2]);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * 16 * TM + i * 16 + r;
      const f32x4& X = acc[2 * p][i];
      const f32x4& Y = acc[2 * p + 1][i];
      const uint32_t x0 = (uint32_t)f32_to_bf16(X[0]) | ((uint32_t)f32_to_bf16(X[1]) << 16);
      const uint32_t x1 = (uint32_t)f32_to_bf16(X[2]) | ((uint32_t)f32_to_bf16(X[3]) << 16);
      const uint32_t y0 = (uint32_t)f32_to_bf16(Y[0]) | ((uint32_t)f32_to_bf16(Y[1]) << 16);
      const uint32_t y1 = (uint32_t)f32_to_bf16(Y[2]) | ((uint32_t)f32_to_bf16(Y[3]) << 16);
      // rows 2q + 1 of the first operand trade places with rows 2q of the second
      const auto s0 = __builtin_amdgcn_permlane16_swap(x0, y0, false, false);
      const auto s1 = __builtin_amdgcn_permlane16_swap(x1, y1, false, false);
      const u32x4v v = {s0[0], s1[0], s0[1], s1[1]};
      if (m < a.M && n < a.Ntot) __builtin_nontemporal_store(v, reinterpret_cast<u32x4v*>(o + (int64_t)m * ld + loc));
    }
  }
}

// SwiGLU output of a bf16 tile (the fused gate/up GEMM): MFMA column tiles j < TN/2 of a wave hold
// W_gate rows and tiles j + TN/2 the W_up rows of the same output features, so lane (r, g) holds
// gate and up of features f .. f + 3 (f = the wave's first feature + 16 j + 4 g) for output row r
// of each row tile and writes h = round(round(silu(round(gate))) * round(up)) as 8 bytes: the eager
// path's rounding points (two GEMM outputs in bf16, silu rounded, the product rounded) and
// dh_silu_mul's bf16 arithmetic (silu with the hardware exp: equal to torch's bf16 SiLU for every
// bf16 input, and 12 instructions per element fewer in an epilogue that runs while the matrix
// cores wait).
template <int TM, int TN, int WGM>
__device__ __forceinline__ void store_tile_swiglu(const GemmArgs& a, const f32x4 (&acc)[TN][TM], int m0, int n0,
                                                  int wm, int wn, int r, int g) {
  static_assert(TN % 2 == 0, "gate and up column tiles in pairs");
  bf16_t* o = (bf16_t*)a.out[0];
  const int64_t ld = a.ldo[0];
  auto out = [&](auto silu) {
#pragma unroll
    for (int p = 0; p < TN / 2; ++p) {
      const int f = n0 / 2 + wn * 8 * TN + p * 16 + 4 * g;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm * 16 * TM + i * 16 + r;
        const f32x4& G = acc[p][i];
        const f32x4& U = acc[p + TN / 2][i];
        float h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          h[e] = Elem<bf16_t>::round(Elem<bf16_t>::round(silu(Elem<bf16_t>::round(G[e]))) * Elem<bf16_t>::round(U[e]));
        const uint32_t lo = (uint32_t)f32_to_bf16(h[0]) | ((uint32_t)f32_to_bf16(h[1]) << 16);
        const uint32_t hi = (uint32_t)f32_to_bf16(h[2]) | ((uint32_t)f32_to_bf16(h[3]) << 16);
        if (m < a.M && f < a.N[0]) *reinterpret_cast<uint2*>(o + (int64_t)m * ld + f) = make_uint2(lo, hi);
      }
    }
  };
  // the reciprocal form unless some gate output of the wave's tile is below -87 (one uniform branch)
  float gmin = 0.f;
#pragma unroll
  for (int p = 0; p < TN / 2; ++p)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) gmin = fminf(gmin, acc[p][i][e]);
  if (__builtin_amdgcn_ballot_w64(gmin < -87.0f))
    out([](float x) { return dh_silu_bf16in(x); });
  else
    out([](float x) { return dh_silu_bf16in_rcp(x); });
}

// Fragment ping-pong variant (bf16, S LDS stages: S - 1 K tiles in flight while one is multiplied;
// the persistent form and well-occupied launches use two): the MFMA operands of a K tile's two 32-k steps
// live in two register sets, so the LDS reads of one step are in flight while the MFMAs of the other
// run, across the K-tile boundary too: the barrier sits between the two steps' MFMAs. Row swizzle:
// slot p of row R holds chunk p ^ (R & 7). Measured with the LDS counters on MI355X, the fragment
// reads (16 lanes = 16 consecutive rows, one chunk; ds_read_b128) then take 4 LDS cycles per
// instruction, the conflict-free minimum, where (R & 7) ^ ((R >> 3) & 1) or a 144-byte row pitch
// take 8. For the fragment rows base + 16 j + r (base a multiple of 16) it depends on r alone, so a
// lane's fragment addresses are one register per step plus immediate offsets. The loads take a
// scalar base (operand + K offset; a weight segment is uniform over a wave's 8-row group when every
// segment width is a multiple of 8) and 32-bit lane offsets.
__device__ __forceinline__ int swz2(int R) { return R & 7; }

// M0 (the LDS destination base) is an input operand bound to the register itself ("{m0}"), so the
// compiler writes it and knows its value is live across the statement; nothing here clobbers a
// register the compiler reserves.
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// SWI: the fused SwiGLU GEMM (segments 0 = W_gate, 1 = W_up, both N[0] rows): column tile nt covers
// output features [nt BN / 2, (nt + 1) BN / 2), each wave's 16 TN columns the gate rows then the
// up rows of its 8 TN features, and the epilogue is store_tile_swiglu.
template <int TM, int TN, int WGM, int WGN, bool SWI, int S>
__global__ __launch_bounds__(64 * WGM * WGN) void proj_gemm_pp_kernel(GemmArgs a) {
  typedef bf16_t T;
  typedef Frag<T> F;
  constexpr int NW = WGM * WGN;
  constexpr int BM = 16 * TM * WGM, BN = 16 * TN * WGN;
  constexpr int GX = BM / 8 / NW, GW = BN / 8 / NW;    // 8-row load groups per wave and operand
  static_assert(GX * 8 * NW == BM && GW * 8 * NW == BN, "tile rows must split into 8-row groups per wave");
  static_assert(F::KSTEPS == 2, "two 32-k steps per 128-byte K tile");
  static_assert(S >= 2, "at least two LDS stages");
  constexpr int PER = GX + GW;                         // DMA instructions per K tile and wave
  __shared__ __align__(1024) unsigned char sw[S][BN * kRowBytes];   // weight tiles
  __shared__ __align__(1024) unsigned char sx[S][BM * kRowBytes];   // activation tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int wm = wave % WGM, wn = wave / WGM;
  const int nk = a.K / 64;
  const int nvirt = ((a.mtiles + 7) / 8) * 8 * a.ntiles;

  // fragment byte offsets within a stage: row R = quadrant base + 16 j + r, chunk 4 ks + g
  const int fw = (wn * 16 * TN + r) * kRowBytes, fx = (wm * 16 * TM + r) * kRowBytes;
  const int sr = swz2(r);
  const int c0 = (g ^ sr) << 4, c1 = ((4 + g) ^ sr) << 4;
  auto read = [&](uint4 (&wf)[TN], uint4 (&xf)[TM], int st, int cofs) {
#pragma unroll
    for (int j = 0; j < TN; ++j) wf[j] = *reinterpret_cast<const uint4*>(&sw[st][fw + j * 16 * kRowBytes + cofs]);
#pragma unroll
    for (int i = 0; i < TM; ++i) xf[i] = *reinterpret_cast<const uint4*>(&sx[st][fx + i * 16 * kRowBytes + cofs]);
  };
  f32x4 acc[TN][TM];
  auto mma_all = [&](const uint4 (&wf)[TN], const uint4 (&xf)[TM]) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) F::mma(acc[j][i], wf[j], xf[i]);
  };

  // load group q of this wave: rows 8G .. 8G+7, G = NW q + wave; lane -> row 8G + lane / 8 whose
  // slot lane % 8 takes chunk (lane % 8) ^ swz2(row); byte offsets from the operand base
  uint32_t xo[GX], wo[GW];
  int wsg[GW];
  auto issue = [&](int kt, int st) {
    const int kb = kt * kRowBytes;
#pragma unroll
    for (int q = 0; q < GW; ++q)
      dma16s((const char*)pick(wsg[q], a.W[0], a.W[1], a.W[2]) + kb, wo[q], lds_addr(&sw[st][(NW * q + wave) * 1024]));
#pragma unroll
    for (int q = 0; q < GX; ++q) dma16s((const char*)a.X + kb, xo[q], lds_addr(&sx[st][(NW * q + wave) * 1024]));
  };
  uint4 aw[TN], ax[TM], bw[TN], bx[TM];                // step-0 and step-1 operand sets
  int pm0 = -1, pn0 = 0;                               // the tile whose output acc holds
  for (int id = blockIdx.x; id < nvirt; id += gridDim.x) {
    const int xcd = id & 7, slot = id >> 3;
    const int mt = (slot / a.ntiles) * 8 + xcd, nt = slot % a.ntiles;
    if (mt >= a.mtiles) continue;                      // uniform
    const int m0 = mt * BM, n0 = nt * BN;
#pragma unroll
    for (int q = 0; q < GX; ++q) {
      const int R = 8 * (NW * q + wave) + (lane >> 3);
      const int m = min(m0 + R, a.M - 1);
      xo[q] = ((uint32_t)m * (uint32_t)a.ldx + (uint32_t)(((lane & 7) ^ swz2(R)) * 8)) * 2u;
    }
#pragma unroll
    for (int q = 0; q < GW; ++q) {
      const int R = 8 * (NW * q + wave) + (lane >> 3);
      int loc;
      if constexpr (SWI) {
        // tile row R = wave column wc, MFMA column tile j, row rr: gate (j < TN/2) or up row of
        // feature n0/2 + 8 TN wc + 16 (j mod TN/2) + rr (an 8-row group lies in one 16-row tile)
        const int wc = R / (16 * TN), j = (R / 16) % TN, rr = R % 16;
        loc = min(n0 / 2 + 8 * TN * wc + 16 * (j % (TN / 2)) + rr, a.N[0] - 1);
        wsg[q] = __builtin_amdgcn_readfirstlane(j < TN / 2 ? 0 : 1);
      } else {
        const int n = min(n0 + R, a.Ntot - 1);
        wsg[q] = __builtin_amdgcn_readfirstlane(seg_of(a, n, loc));
      }
      wo[q] = ((uint32_t)loc * (uint32_t)a.K + (uint32_t)(((lane & 7) ^ swz2(R)) * 8)) * 2u;
    }
    __syncthreads();                                   // the previous tile's LDS reads are done
    issue(0, 0);
#pragma unroll
    for (int q = 1; q + 1 < S; ++q) issue(min(q, nk - 1), q);
    const bool first = pm0 < 0;                        // uniform: no output of this workgroup yet
    if (!first) {                                      // under K tile 0's loads
      if constexpr (SWI) store_tile_swiglu<TM, TN, WGM>(a, acc, pm0, pn0, wm, wn, r, g);
      else store_tile_x4<TM, TN, WGM>(a, acc, pm0, pn0, wm, wn, r, g);
    }
    pm0 = m0;
    pn0 = n0;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    // K tile 0 has landed: in a workgroup's first tile only loads are in flight and they complete in
    // issue order, so tiles 1 .. S-2 may still be on their way; after an output, everything
    if (first) wait_vm<(S - 2) * PER>();
    else wait_vm<0>();
    __syncthreads();
    issue(min(S - 1, nk - 1), S - 1);
    read(aw, ax, 0, c0);
    int st = 0;                                        // stage of tile kt: kt mod S
    for (int kt = 0; kt < nk; ++kt) {
      const int nst = st + 1 == S ? 0 : st + 1;
      read(bw, bx, st, c1);                            // step 1 of tile kt ...
      mma_all(aw, ax);                                 // ... in flight under step 0's MFMAs
      // Scheduling fences: without them the compiler sinks step 0's MFMAs below the barrier (they
      // touch no memory), which leaves step 1's reads waited on with nothing in flight under them.
      __builtin_amdgcn_sched_barrier(0);
      // tile kt + 1 has landed (this wave's part): loads complete in issue order, and the S - 2
      // tiles issued after it may still be in flight
      wait_vm<(S - 2) * PER>();
      __syncthreads();                                 // everyone's; every read of stage st is done
      issue(min(kt + S, nk - 1), st);                  // (repeats of the last tile are harmless)
      if (kt + 1 < nk) read(aw, ax, nst, c0);          // step 0 of tile kt + 1 ...
      __builtin_amdgcn_sched_barrier(0);
      mma_all(bw, bx);                                 // ... under step 1's MFMAs
      __builtin_amdgcn_sched_barrier(0);
      st = nst;
    }
    wait_vm<0>();                                      // repeated tail loads land before LDS is reused
  }
  if (pm0 >= 0) {
    if constexpr (SWI) store_tile_swiglu<TM, TN, WGM>(a, acc, pm0, pn0, wm, wn, r, g);
    else store_tile_x4<TM, TN, WGM>(a, acc, pm0, pn0, wm, wn, r, g);
  }
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

// One workgroup per tile of the ping-pong kernel with 4 waves (BM = 32 TM, BN = 32 TN), S LDS stages.
template <int TM, int TN, bool SWI, int S = 2>
int launch_pp_tiles(GemmArgs& a, hipStream_t s, const char* who) {
  constexpr int BM = 32 * TM, BN = 32 * TN;
  a.mtiles = (a.M + BM - 1) / BM;
  a.ntiles = (a.Ntot + BN - 1) / BN;
  const int64_t nvirt = (int64_t)((a.mtiles + 7) / 8) * 8 * a.ntiles;
  DH_REQUIRE(nvirt < (1ll << 31), DH_ERR_UNSUPPORTED_SHAPE, "%s: M=%d too large", who, a.M);
  proj_gemm_pp_kernel<TM, TN, 2, 2, SWI, S><<<dim3((unsigned)nvirt), dim3(256), 0, s>>>(a);
  return dh_check_launch(who);
}

int64_t tiles_of(int M, int N, int BM, int BN) { return (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN); }

constexpr int64_t kWideMinTiles = 160;    // 256 x 256 tiles from ~0.6 per CU (persistent, one per CU)
constexpr int64_t kWideGrid = 256;        // persistent workgroups: one per CU (128 KB of LDS each)

// The ping-pong kernel's tile for M x Ntot (Ntot: concatenated output columns; the fused SwiGLU
// GEMM's gate and up rows count both). Measured on MI355X in captured graphs, bf16, K = 1024
// unless noted (us; 64x64 / 64x128 / 128x64 / 128x128 / 256x256):
//   M = 1024  N = 3072          13.6 / 14.7 / 14.3 / 16.4 / 28.0
//   M = 1024  N = 2 x 2816      28.4 / 21.6 / 21.5 / 21.7 / 28.8
//   M = 2048  N = 3072          26.1 / 19.6 / 19.8 / 19.6 / 27.8
//   M = 2048  N = 2 x 2816      51.4 / 42.4 / 39.9 / 37.1 / 30.6
//   M = 4096  N = 3072          49.3 / 40.1 / 38.9 / 36.9 / 30.0
//   M = 4096  N = 1024          14.7 / 13.3 / 12.7 / 15.7 / 26.0
//   M = 4096  N = 1024 K = 2816 38.8 / 30.0 / 29.8 / 34.1 / 62.3
// i.e. 256 x 256 tiles from ~160 of them, else 64 x 64 while there are at most 768 of those (three
// per CU), else the largest count of 64 x 128 (>= 768) or 128 x 64 (>= 512) tiles, else 128 x 128.
// With at most one or two 64 x 64 tiles per CU nothing else on the CU covers a K tile's round trip,
// so those launches keep three (<= 256 tiles) or two (<= 512) K tiles in flight in four or three
// LDS stages instead of one in two. Measured over 18 distinct weights per graph (us, two / three /
// four stages): M = 1024 N = 1024 9.8 / 7.1 / 6.7, M = 1024 N = 1024 K = 2816 21.7 / 13.5 / 12.1,
// M = 2048 N = 1024 10.4 / 9.1 / 9.6, M = 2048 N = 1024 K = 2816 22.3 / 19.8 / 20.4; with more tiles
// per CU the extra LDS costs occupancy (M = 1024 N = 3072: 12.6 / 14.3 / 16.3).
// Every form sums the same products in the same k order: outputs are bit-identical across forms
// and stage counts.
template <bool SWI>
int launch_wide(GemmArgs& a, hipStream_t s, const char* who) {
  const int M = a.M, N = a.Ntot;
  if (tiles_of(M, N, 256, 256) >= kWideMinTiles) {
    a.mtiles = (M + 255) / 256;
    a.ntiles = (N + 255) / 256;
    const int64_t nvirt = (int64_t)((a.mtiles + 7) / 8) * 8 * a.ntiles;
    DH_REQUIRE(nvirt < (1ll << 31), DH_ERR_UNSUPPORTED_SHAPE, "%s: M=%d too large", who, M);
    const unsigned grid = (unsigned)(nvirt < kWideGrid ? nvirt : kWideGrid);
    proj_gemm_pp_kernel<8, 4, 2, 4, SWI, 2><<<dim3(grid), dim3(512), 0, s>>>(a);
    return dh_check_launch(who);
  }
  const int64_t t64 = tiles_of(M, N, 64, 64);
  if (t64 <= 256) return launch_pp_tiles<2, 2, SWI, 4>(a, s, who);
  if (t64 <= 512) return launch_pp_tiles<2, 2, SWI, 3>(a, s, who);
  if (t64 <= 768) return launch_pp_tiles<2, 2, SWI>(a, s, who);
  if (tiles_of(M, N, 64, 128) >= 768) return launch_pp_tiles<2, 4, SWI>(a, s, who);
  if (tiles_of(M, N, 128, 64) >= 512) return launch_pp_tiles<4, 2, SWI>(a, s, who);
  return launch_pp_tiles<4, 4, SWI>(a, s, who);
}

}  // namespace

extern "C" int dh_proj_gemm(int dtype, const void* X, int64_t ldx, int M, int K, int nseg, const void* const* W,
                            const int* N, void* const* out, const int64_t* ldo, void* stream) {
  const char* who = "dh_proj_gemm";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(nseg >= 1 && nseg <= 3, DH_ERR_INVALID_ARG, "%s: nseg=%d not in [1,3]", who, nseg);
  DH_REQUIRE(X && W && N && out && ldo, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  const int esz = dtype == DH_BF16 ? 2 : 4;
  const int kt = kRowBytes / esz;
  DH_REQUIRE(M >= 1 && K >= kt && K % kt == 0, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: M=%d K=%d (K must be a positive multiple of %d)", who, M, K, kt);
  DH_REQUIRE(ldx >= K && aligned(X, 16) && (ldx * esz) % 16 == 0, DH_ERR_INVALID_ARG,
             "%s: X rows need ldx >= K and 16-byte alignment", who);
  GemmArgs a{};
  a.X = X;
  a.ldx = ldx;
  a.nseg = nseg;
  a.M = M;
  a.K = K;
  int total = 0;
  for (int s = 0; s < nseg; ++s) {
    DH_REQUIRE(W[s] && out[s] && N[s] >= 4 && N[s] % 4 == 0, DH_ERR_INVALID_ARG,
               "%s: segment %d needs weights, an output and N a positive multiple of 4", who, s);
    DH_REQUIRE(aligned(W[s], 16) && aligned(out[s], 4 * esz) && ldo[s] >= N[s] && ldo[s] % 4 == 0,
               DH_ERR_INVALID_ARG, "%s: segment %d alignment / leading dimension", who, s);
    a.W[s] = W[s];
    a.out[s] = out[s];
    a.ldo[s] = ldo[s];
    a.N[s] = N[s];
    total += N[s];
  }
  a.Ntot = total;
  hipStream_t s = (hipStream_t)stream;
  // bf16 launches whose operands and outputs meet the ping-pong kernels' conditions (32-bit operand
  // offsets, segment widths multiples of 8, 16-byte aligned output rows) take them (launch_wide);
  // the rest (fp32 among them) the 128 x 128 register-staged kernel.
  bool wide = dtype == DH_BF16 && (int64_t)M * ldx * esz < (1ll << 31);
  for (int i = 0; i < nseg; ++i)
    wide = wide && N[i] % 8 == 0 && (int64_t)N[i] * K * esz < (1ll << 31) && ldo[i] % 8 == 0 && aligned(out[i], 16);
  if (wide) return launch_wide<false>(a, s, who);
  a.mtiles = (M + kBM - 1) / kBM;
  a.ntiles = (total + kBN - 1) / kBN;
  const int64_t grid = (int64_t)((a.mtiles + 7) / 8) * 8 * a.ntiles;
  DH_REQUIRE(grid < (1ll << 31), DH_ERR_UNSUPPORTED_SHAPE, "%s: M=%d too large", who, M);
  if (dtype == DH_BF16)
    proj_gemm_kernel<bf16_t><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(a);
  else
    proj_gemm_kernel<float><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(a);
  return dh_check_launch(who);
}

// out[m, f] = round(round(silu(round(X[m] . Wg[f]))) * round(X[m] . Wu[f])): a SwiGLU layer's
// gate and up GEMMs and its activation (reference dispatcher_hybrid/modeling_dispatcher.py:188-197,
// F.silu(linear_gate(h)) * linear_up(h)) as one launch of the ping-pong kernel over the 2N
// concatenated weight rows, bf16 only. Without it: two GEMMs writing gate and up to memory, then
// dh_silu_mul reading them back.
extern "C" int dh_proj_gemm_swiglu(int dtype, const void* X, int64_t ldx, int M, int K, const void* Wg,
                                   const void* Wu, int N, void* out, int64_t ldo, void* stream) {
  const char* who = "dh_proj_gemm_swiglu";
  DH_REQUIRE(dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d (bf16 only)", who, dtype);
  DH_REQUIRE(X && Wg && Wu && out, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(M >= 1 && K >= 64 && K % 64 == 0 && N >= 8 && N % 8 == 0, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: M=%d K=%d N=%d (K a positive multiple of 64, N of 8)", who, M, K, N);
  DH_REQUIRE(ldx >= K && ldx % 8 == 0 && aligned(X, 16) && aligned(Wg, 16) && aligned(Wu, 16) &&
                 ldo >= N && ldo % 8 == 0 && aligned(out, 16),
             DH_ERR_INVALID_ARG, "%s: operands need 16-byte aligned rows (ldx >= K, ldo >= N)", who);
  DH_REQUIRE((int64_t)M * ldx * 2 < (1ll << 31) && (int64_t)N * K * 2 < (1ll << 31), DH_ERR_UNSUPPORTED_SHAPE,
             "%s: operands past 2 GB", who);
  GemmArgs a{};
  a.X = X;
  a.ldx = ldx;
  a.nseg = 2;
  a.M = M;
  a.K = K;
  a.W[0] = Wg;
  a.W[1] = Wu;
  a.out[0] = out;
  a.ldo[0] = ldo;
  a.N[0] = a.N[1] = N;
  a.Ntot = 2 * N;
  return launch_wide<true>(a, (hipStream_t)stream, who);
}
