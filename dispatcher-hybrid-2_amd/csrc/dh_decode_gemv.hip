// Decode-step matrix-vector products with their neighbouring elementwise work fused in, for gfx950.
//
// One launch computes, for each batch row b and output row n of up to three concatenated weight
// segments W_s (N_s x K, row-major, in the model dtype):
//     h      = RMSNorm(x[b]) * g            (optional prologue; fp32 math, rounded to the dtype)
//     acc    = W_s[n] . h                   (fp32 accumulation)
//     out    = round(acc)                                     plain
//            | round(round(acc) + resid[b, n])                residual add (segment 0 only)
//            | round(round(silu(round(acc_gate))) * round(acc_up))   SwiGLU (segments gate, up)
// and writes out to segment s's destination at b * out_bstride + t * t_stride + n (t = the device
// position, for the B_hist[t] row of the mixer's source projection). The rounding points are those
// of the eager torch step (reference dispatcher_hybrid/decoding.py:473-476 and :487-488,
// dispatcher_hybrid/modeling_dispatcher.py:196-197, 207-212, 348-351).
//
// Work decomposition: every wave works alone (no LDS, no barriers). A wave owns R consecutive
// output rows; lane l owns the 16-byte chunks l, l+64, ... of K in each of them and loads its
// weight chunks, the matching chunks of the activation rows and of the RMSNorm weight straight
// from memory, all before any arithmetic (no load is guarded by a divergent branch: addresses are
// clamped and predicates applied to values). Since the wave's lanes cover the whole row, the wave
// computes the RMSNorm sum of squares itself with one DPP wave reduction, then each (row, batch
// row) dot product with another; every lane then holds every sum and lane j writes output j. R is
// 1 except for very tall matrices, so a launch keeps several thousand waves, and their loads, in
// flight: for these small matrices the time is set by how many loads are outstanding, not by the
// bytes.
#include "dh_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSeg = 3;

struct Seg {
  const void* W;
  void* out;
  int64_t out_bstride;
  int64_t t_stride;
  int N;
};

struct GemvArgs {
  const void* x;
  int64_t x_bstride;
  const int64_t* x_rows;        // nullable: x row of batch b is x_rows[b] (embedding gather)
  const void* g;                // nullable RMSNorm weight (K)
  float eps;
  const void* resid;            // nullable residual (B, N0)
  int64_t resid_bstride;
  const int64_t* resid_rows;    // nullable: residual row of batch b is resid_rows[b]
  const int64_t* t_dev;         // device position (read only when some segment has a t_stride)
  int64_t* t_advance;           // nullable: incremented by one by this launch
  int uses_t;
  Seg seg[kMaxSeg];
  int nseg;
  int B, K, Nrows;
  Cand* cand;                   // nullable (B = 1): the launch's argmax candidate per workgroup
  int tile_rows;                // batched matrix-core GEMV: real weight rows per 16-row MFMA tile (16 or 8)
  // batched matrix-core GEMV, 16-row MFMA fragment order (16-byte chunk (s * 64 + 16 g + r) holds
  // row r's elements s * 32 + 8 g .. + 7): frag_out writes the outputs so (a SwiGLU launch's h),
  // frag_in reads the activations so, one contiguous 1 KB per wave and k-step
  int frag_out, frag_in;
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Weight rows are streamed once per decode step: their loads carry the non-temporal hint, so they do
// not push out of L2 the small state the step reads back (ring slots, history rows, activations).
// Measured: batch-16 step 0.667 -> 0.660 ms, the one-launch batch-1 step 337.3 -> 335.8 us.
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldw16(const void* p) {
  const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <typename T> struct Vec;
template <> struct Vec<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static uint4 pack(const float (&o)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (uint32_t)f32_to_bf16(o[2 * j]) | ((uint32_t)f32_to_bf16(o[2 * j + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ __forceinline__ static void unpack(const uint4& v, float (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = __uint_as_float(w[j] << 16);
      o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
};
template <> struct Vec<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static uint4 pack(const float (&o)[4]) {
    return make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3]));
  }
  __device__ __forceinline__ static void unpack(const uint4& v, float (&o)[4]) {
    o[0] = __uint_as_float(v.x);
    o[1] = __uint_as_float(v.y);
    o[2] = __uint_as_float(v.z);
    o[3] = __uint_as_float(v.w);
  }
};

__device__ __forceinline__ float silu(float x) { return x * dh_sigmoid(x); }

// raw element bits: the conversion (the load's first consumer) can sit after the whole burst
template <typename T> struct Raw;
template <> struct Raw<bf16_t> {
  __device__ __forceinline__ static uint32_t load(const bf16_t* p) { return *p; }
  __device__ __forceinline__ static float f(uint32_t r) { return __uint_as_float(r << 16); }
};
template <> struct Raw<float> {
  __device__ __forceinline__ static uint32_t load(const float* p) { return __float_as_uint(*p); }
  __device__ __forceinline__ static float f(uint32_t r) { return __uint_as_float(r); }
};

// Raw buffer access: a descriptor (base, byte range) in scalar registers and a per-lane byte offset;
// a read past the range returns zeros without a memory request. dword3 = 0x00020000 is the
// gfx9-family raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
constexpr int kNT = 2;                                 // buffer-load cache policy: non-temporal
__device__ __forceinline__ uint4 bld16w(__amdgpu_buffer_rsrc_t r, uint32_t voff) {   // weight rows
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kNT));
}
__device__ __forceinline__ uint32_t bld2(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
}

// Segment of concatenated output row n, from uniform selects over the argument fields (indexing
// the argument array with a runtime value makes the compiler read it with vector loads, and wait
// for them, before the weight requests).
struct RowSeg {
  int s, local;
};
__device__ __forceinline__ RowSeg row_segment(const GemvArgs& a, int n) {
  const int N0 = a.seg[0].N, N1 = a.seg[1].N;
  const bool in1 = a.nseg > 1 && n >= N0;
  const bool in2 = a.nseg > 2 && n >= N0 + N1;
  return RowSeg{in2 ? 2 : (in1 ? 1 : 0), n - (in2 ? N0 + N1 : (in1 ? N0 : 0))};
}
template <typename P>
__device__ __forceinline__ P pick_seg(int s, P p0, P p1, P p2) {
  return s == 0 ? p0 : (s == 1 ? p1 : p2);
}
// destination of output `loc` of segment s for batch row b at position t
template <typename T>
__device__ __forceinline__ T* out_ptr(const GemvArgs& a, int s, int64_t b, int64_t t, int loc) {
  T* o = (T*)pick_seg(s, a.seg[0].out, a.seg[1].out, a.seg[2].out);
  return o + b * pick_seg(s, a.seg[0].out_bstride, a.seg[1].out_bstride, a.seg[2].out_bstride) +
         t * pick_seg(s, a.seg[0].t_stride, a.seg[1].t_stride, a.seg[2].t_stride) + loc;
}

// the launch's position advance (block 0, thread 0), placed after the launch's requests
__device__ __forceinline__ void advance_position(const GemvArgs& a) {
  if (a.t_advance && blockIdx.x == 0 && threadIdx.x == 0) *a.t_advance += 1;   // host: uses_t == 0
}

template <typename T, int R, int CG, int BG, bool SW>
__global__ __launch_bounds__(kThreads) void decode_gemv_kernel(GemvArgs a) {
  constexpr int V = Vec<T>::N;
  constexpr int NW = SW ? 2 : 1;                      // weight rows per output row
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.K, B = a.B;
  const int nchunk = K / V;
  const bool has_norm = a.g != nullptr;
  const int rbase = (blockIdx.x * kWaves + wave) * R;
  // (no early exit for waves past the last row: a branch here would make every wave wait for the
  // row count before requesting anything; their loads are clamped and their stores predicated;
  // the position advance, when asked for, comes last for the same reason)

  // ---- weights: every load of the wave in one burst
  const T* wrow[R][NW];
  int segi[R];
  int local[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(rbase + r, a.Nrows - 1);
    const RowSeg rw = SW ? RowSeg{0, n} : row_segment(a, n);
    segi[r] = rw.s;
    local[r] = rw.local;
    wrow[r][0] = (const T*)pick_seg(rw.s, a.seg[0].W, a.seg[1].W, a.seg[2].W) + (int64_t)rw.local * K;
    if (SW) wrow[r][NW - 1] = (const T*)a.seg[1].W + (int64_t)rw.local * K;
  }
  uint4 w[R][NW][CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int ch = min(lane + 64 * c, nchunk - 1);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q) w[r][q][c] = ldw16(wrow[r][q] + (int64_t)ch * V);
  }
  uint4 gv[CG];
  if (has_norm) {                                      // uniform
#pragma unroll
    for (int c = 0; c < CG; ++c) gv[c] = ld16((const T*)a.g + (int64_t)min(lane + 64 * c, nchunk - 1) * V);
  }
  const int64_t t = a.uses_t ? load_uniform(a.t_dev) : 0;
  const bool has_resid = a.resid != nullptr;

  // activation chunks of BG batch rows (gathered through x_rows when given) and the residual
  // operand of the output this lane writes (output j = lane: row j % R, batch row b0 + j / R).
  // The first group is requested in the same burst as the weights and each later group while the
  // previous one is computed, so no load waits for another one (the weight unpacking, which the
  // compiler hoists out of the batch loop, comes after these requests).
  uint4 xv[BG][CG];
  uint32_t resid_raw = 0;
  auto fetch_group = [&](int g0) {
#pragma unroll
    for (int bp = 0; bp < BG; ++bp) {
      const int b = min(g0 + bp, B - 1);
      const int64_t xrow = a.x_rows ? load_uniform(a.x_rows + b) : (int64_t)b;
      const T* xp = (const T*)a.x + xrow * a.x_bstride;
#pragma unroll
      for (int c = 0; c < CG; ++c) xv[bp][c] = ld16(xp + (int64_t)min(lane + 64 * c, nchunk - 1) * V);
    }
    if (has_resid) {                                   // uniform
      const int b = min(g0 + lane / R, B - 1);
      const int n = min(rbase + lane % R, a.Nrows - 1);
      const int64_t rrow = a.resid_rows ? a.resid_rows[b] : (int64_t)b;
      resid_raw = Raw<T>::load((const T*)a.resid + rrow * a.resid_bstride + n);
    }
  };
  fetch_group(0);

  for (int b0 = 0; b0 < B; b0 += BG) {
    uint4 xc[BG][CG];
#pragma unroll
    for (int bp = 0; bp < BG; ++bp)
#pragma unroll
      for (int c = 0; c < CG; ++c) xc[bp][c] = xv[bp][c];
    const uint32_t rc = resid_raw;
    if (b0 + BG < B) fetch_group(b0 + BG);             // uniform; used in the next iteration
    // ---- RMSNorm scale of each batch row: the wave's lanes cover the whole row
    float rs[BG];
#pragma unroll
    for (int bp = 0; bp < BG; ++bp) {
      rs[bp] = 1.f;
      if (has_norm) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          float xf[V];
          Vec<T>::unpack(xc[bp][c], xf);
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < V; ++e) part += xf[e] * xf[e];
          ss += lane + 64 * c < nchunk ? part : 0.f;
        }
        rs[bp] = rsqrtf(wave_sum(ss) / (float)K + a.eps);
      }
    }
    // ---- dot products
    float acc[R][NW][BG];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q)
#pragma unroll
        for (int bp = 0; bp < BG; ++bp) acc[r][q][bp] = 0.f;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const bool live = lane + 64 * c < nchunk;
      float gw[V];
      if (has_norm) Vec<T>::unpack(gv[c], gw);
#pragma unroll
      for (int bp = 0; bp < BG; ++bp) {
        float hv[V];
        Vec<T>::unpack(xc[bp][c], hv);
        if (has_norm) {
#pragma unroll
          for (int e = 0; e < V; ++e) hv[e] = Elem<T>::round(hv[e] * rs[bp] * gw[e]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int q = 0; q < NW; ++q) {
            float wv[V];
            Vec<T>::unpack(w[r][q][c], wv);
            float sdot = 0.f;
#pragma unroll
            for (int e = 0; e < V; ++e) sdot += wv[e] * hv[e];
            acc[r][q][bp] += live ? sdot : 0.f;
          }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q)
#pragma unroll
        for (int bp = 0; bp < BG; ++bp) acc[r][q][bp] = wave_sum(acc[r][q][bp]);
    // ---- epilogue: lane j writes output (row j % R, batch row b0 + j / R)
    const int r = lane % R, bp = lane / R;
    if (bp < BG && b0 + bp < B && rbase + r < a.Nrows) {
      float v0 = 0.f, v1 = 0.f;
#pragma unroll
      for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int pp = 0; pp < BG; ++pp)
          if (rr == r && pp == bp) {
            v0 = acc[rr][0][pp];
            v1 = acc[rr][NW - 1][pp];
          }
      float out;
      if (SW) {
        out = Elem<T>::round(Elem<T>::round(silu(Elem<T>::round(v0))) * Elem<T>::round(v1));
      } else {
        out = Elem<T>::round(v0);
        if (has_resid) out = Elem<T>::round(out + Raw<T>::f(rc));
      }
      int s = 0, loc = 0;
#pragma unroll
      for (int rr = 0; rr < R; ++rr)
        if (rr == r) {
          s = segi[rr];
          loc = local[rr];
        }
      Elem<T>::store(out_ptr<T>(a, s, b0 + bp, t, loc), out);
    }
  }
  advance_position(a);
}

// Single-row variant (B == 1). Every lane of the per-wave kernel above requests its own copy of
// the activation row and of the RMSNorm weight: three requests per weight request, all through
// the compute unit's vector memory path, which bounds these short launches. Here each workgroup
// requests the two rows once, one 16-byte load per thread, stages them in LDS behind one barrier,
// normalises the row once (block sum of squares, then the scaled row written back in place), and
// each wave reads its chunks from LDS. The small requests (activation, norm weight, residual)
// go out BEFORE the weight burst: loads return in issue order, so they arrive first and the
// staging never waits for the weights. When a row is gathered through x_rows or resid_rows (the
// embedding), its address waits on a scalar load, so the weights go first instead (GATHER).
// Same arithmetic as the per-wave kernel.
template <typename T, int R, int CG, bool SW, int NT, bool GATHER>
__global__ __launch_bounds__(NT) void decode_gemv_row_kernel(GemvArgs a) {
  __shared__ uint4 sx[2 * CG * 64];                   // x chunks [0, nchunk), norm weight after
  constexpr int V = Vec<T>::N;
  constexpr int NW = SW ? 2 : 1;
  constexpr int NWV = NT / 64;
  constexpr int XCH = (2 * CG * 64 + NT - 1) / NT;     // staged chunks per thread
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.K;
  const int nchunk = K / V;
  const bool has_norm = a.g != nullptr;
  const bool has_resid = a.resid != nullptr;
  const int nst = has_norm ? 2 * nchunk : nchunk;
  const int rbase = (blockIdx.x * NWV + wave) * R;

  uint4 st[XCH];
  uint32_t rc = 0;
  auto small_loads = [&]() {
    const int64_t xrow = GATHER && a.x_rows ? load_uniform(a.x_rows) : 0;
    const T* xp = (const T*)a.x + xrow * a.x_bstride;
    const T* gp = has_norm ? (const T*)a.g : xp;
#pragma unroll
    for (int j = 0; j < XCH; ++j) {
      const int i = min((int)threadIdx.x + j * NT, nst - 1);
      st[j] = ld16(i < nchunk ? xp + (int64_t)i * V : gp + (int64_t)(i - nchunk) * V);
    }
    // the residual of output `lane`; without one, a harmless read of x keeps the load unconditional
    // (a branch around it makes the no-residual path wait for the staging loads)
    const int n = min(rbase + lane % R, a.Nrows - 1);
    const int64_t rrow = GATHER && a.resid_rows ? load_uniform(a.resid_rows) : 0;
    rc = Raw<T>::load(has_resid ? (const T*)a.resid + rrow * a.resid_bstride + n : xp);
  };
  if constexpr (!GATHER) {
    small_loads();
    DH_ISSUE_FENCE();
  }

  // ---- weights: every load of the wave in one burst
  const T* wrow[R][NW];
  int segi[R];
  int local[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(rbase + r, a.Nrows - 1);
    const RowSeg rw = SW ? RowSeg{0, n} : row_segment(a, n);
    segi[r] = rw.s;
    local[r] = rw.local;
    wrow[r][0] = (const T*)pick_seg(rw.s, a.seg[0].W, a.seg[1].W, a.seg[2].W) + (int64_t)rw.local * K;
    if (SW) wrow[r][NW - 1] = (const T*)a.seg[1].W + (int64_t)rw.local * K;
  }
  uint4 w[R][NW][CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int ch = min(lane + 64 * c, nchunk - 1);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q) w[r][q][c] = ldw16(wrow[r][q] + (int64_t)ch * V);
  }
  if constexpr (GATHER) small_loads();
  const int64_t t = a.uses_t ? load_uniform(a.t_dev) : 0;
  DH_ISSUE_FENCE();

  // ---- stage the activation row; with a norm, the workgroup normalises it once, in place
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < nst) sx[i] = st[j];
  }
  __syncthreads();
  if (has_norm) {                                      // uniform
    __shared__ float red[NWV];
    float ss = 0.f;
    for (int i = threadIdx.x; i < nchunk; i += NT) {
      float xf[V];
      Vec<T>::unpack(sx[i], xf);
#pragma unroll
      for (int e = 0; e < V; ++e) ss += xf[e] * xf[e];
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < NWV; ++w2) tot += red[w2];
    const float rs = rsqrtf(tot / (float)K + a.eps);
    for (int i = threadIdx.x; i < nchunk; i += NT) {
      float xf[V], gw[V];
      Vec<T>::unpack(sx[i], xf);
      Vec<T>::unpack(sx[nchunk + i], gw);
#pragma unroll
      for (int e = 0; e < V; ++e) xf[e] = Elem<T>::round(xf[e] * rs * gw[e]);
      sx[i] = Vec<T>::pack(xf);
    }
    __syncthreads();
  }
  uint4 xc[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) xc[c] = sx[min(lane + 64 * c, nchunk - 1)];

  // ---- dot products
  float acc[R][NW];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < NW; ++q) acc[r][q] = 0.f;
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const bool live = lane + 64 * c < nchunk;
    float hv[V];
    if constexpr (sizeof(T) != 2) Vec<T>::unpack(xc[c], hv);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        float sdot = 0.f;
        if constexpr (sizeof(T) == 2) {
          sdot = dot8_bf16(w[r][q][c], xc[c]);         // as the one-launch step's dot_rows
        } else {
          float wv[V];
          Vec<T>::unpack(w[r][q][c], wv);
#pragma unroll
          for (int e = 0; e < V; ++e) sdot += wv[e] * hv[e];
        }
        acc[r][q] += live ? sdot : 0.f;
      }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < NW; ++q) acc[r][q] = wave_sum(acc[r][q]);
  // ---- epilogue: lane r < R writes output row rbase + r
  float cv = -INFINITY;                                // argmax candidate of this lane (none: -inf)
  int ci = 0x7fffffff;
  if (lane < R && rbase + lane < a.Nrows) {
    float v0 = 0.f, v1 = 0.f;
    int s = 0, loc = 0;
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
      if (rr == lane) {
        v0 = acc[rr][0];
        v1 = acc[rr][NW - 1];
        s = segi[rr];
        loc = local[rr];
      }
    float out;
    if (SW) {
      out = Elem<T>::round(Elem<T>::round(silu(Elem<T>::round(v0))) * Elem<T>::round(v1));
    } else {
      out = Elem<T>::round(v0);
      if (has_resid) {
        uint32_t rv = rc;
        asm volatile("" : "+v"(rv));                    // convert here, not beside the load
        out = Elem<T>::round(out + Raw<T>::f(rv));
      }
    }
    Elem<T>::store(out_ptr<T>(a, s, 0, t, loc), out);
    cv = out;
    ci = rbase + lane;
  }
  if (a.cand) {                                        // uniform: greedy pick fused into the head
    // every output of the workgroup is one (rounded value, row) candidate; the workgroup's best,
    // in torch.argmax's order, goes to cand[blockIdx.x]
    __shared__ Cand wbest[NWV];
    wave_best(cv, ci);
    if (lane == 63) wbest[wave] = Cand{cv, ci};
    __syncthreads();
    if (threadIdx.x == 0) {
      Cand c = wbest[0];
#pragma unroll
      for (int w2 = 1; w2 < NWV; ++w2)
        if (beats(wbest[w2].v, wbest[w2].i, c.v, c.i)) c = wbest[w2];
      a.cand[blockIdx.x] = c;
    }
  }
  advance_position(a);
}

// Batched variant (B > 1): the workgroup normalises each activation row ONCE into LDS (wave w takes
// rows w, w + 4, ...; one barrier), then every wave runs its rows' dot products against the staged
// rows. Same loads-first order: the weight burst is issued before the staging.
template <typename T, int R, int CG, bool SW>
__global__ __launch_bounds__(kThreads) void decode_gemv_staged_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  T* hs = reinterpret_cast<T*>(smem);                 // [B][nchunk * V] staged (normalised) rows
  constexpr int V = Vec<T>::N;
  constexpr int NW = SW ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.K, B = a.B;
  const int nchunk = K / V;
  const bool has_norm = a.g != nullptr;
  const int rbase = (blockIdx.x * kWaves + wave) * R;

  const T* wrow[R][NW];
  int segi[R];
  int local[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(rbase + r, a.Nrows - 1);
    const RowSeg rw = SW ? RowSeg{0, n} : row_segment(a, n);
    segi[r] = rw.s;
    local[r] = rw.local;
    wrow[r][0] = (const T*)pick_seg(rw.s, a.seg[0].W, a.seg[1].W, a.seg[2].W) + (int64_t)rw.local * K;
    if (SW) wrow[r][NW - 1] = (const T*)a.seg[1].W + (int64_t)rw.local * K;
  }
  uint4 w[R][NW][CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int ch = min(lane + 64 * c, nchunk - 1);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q) w[r][q][c] = ldw16(wrow[r][q] + (int64_t)ch * V);
  }
  uint4 gv[CG];
  if (has_norm) {
#pragma unroll
    for (int c = 0; c < CG; ++c) gv[c] = ld16((const T*)a.g + (int64_t)min(lane + 64 * c, nchunk - 1) * V);
  }
  const int64_t t = a.uses_t ? load_uniform(a.t_dev) : 0;

  // ---- staging: wave w normalises rows w, w + 4, ... (its lanes cover the row's chunks)
  for (int b = wave; b < B; b += kWaves) {
    const int64_t xrow = a.x_rows ? load_uniform(a.x_rows + b) : (int64_t)b;
    const T* xp = (const T*)a.x + xrow * a.x_bstride;
    uint4 xv[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) xv[c] = ld16(xp + (int64_t)min(lane + 64 * c, nchunk - 1) * V);
    float rs = 1.f;
    if (has_norm) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        float xf[V];
        Vec<T>::unpack(xv[c], xf);
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < V; ++e) part += xf[e] * xf[e];
        ss += lane + 64 * c < nchunk ? part : 0.f;
      }
      rs = rsqrtf(wave_sum(ss) / (float)K + a.eps);
    }
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const int ch = lane + 64 * c;
      if (ch < nchunk) {
        uint4 hv = xv[c];
        if (has_norm) {
          float xf[V], gw[V];
          Vec<T>::unpack(xv[c], xf);
          Vec<T>::unpack(gv[c], gw);
#pragma unroll
          for (int e = 0; e < V; ++e) xf[e] = xf[e] * rs * gw[e];
          hv = Vec<T>::pack(xf);
        }
        *reinterpret_cast<uint4*>(hs + ((int64_t)b * nchunk + ch) * V) = hv;
      }
    }
  }
  __syncthreads();
  advance_position(a);
  if (rbase >= a.Nrows) return;                       // after the barrier: every wave staged its rows

  // ---- dot products from the staged rows, four batch rows at a time
  constexpr int BG = 4;
  for (int b0 = 0; b0 < B; b0 += BG) {
    const bool has_resid = a.resid != nullptr;
    uint32_t rc = 0;
    if (has_resid) {
      const int b = min(b0 + lane / R, B - 1);
      const int n = min(rbase + lane % R, a.Nrows - 1);
      const int64_t rrow = a.resid_rows ? a.resid_rows[b] : (int64_t)b;
      rc = Raw<T>::load((const T*)a.resid + rrow * a.resid_bstride + n);
    }
    float acc[R][NW][BG];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q)
#pragma unroll
        for (int bp = 0; bp < BG; ++bp) acc[r][q][bp] = 0.f;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const int chr = lane + 64 * c;
      const bool live = chr < nchunk;
      const int ch = min(chr, nchunk - 1);
#pragma unroll
      for (int bp = 0; bp < BG; ++bp) {
        const int b = min(b0 + bp, B - 1);
        float hv[V];
        Vec<T>::unpack(*reinterpret_cast<const uint4*>(hs + ((int64_t)b * nchunk + ch) * V), hv);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int q = 0; q < NW; ++q) {
            float wv[V];
            Vec<T>::unpack(w[r][q][c], wv);
            float sdot = 0.f;
#pragma unroll
            for (int e = 0; e < V; ++e) sdot += wv[e] * hv[e];
            acc[r][q][bp] += live ? sdot : 0.f;
          }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q)
#pragma unroll
        for (int bp = 0; bp < BG; ++bp) acc[r][q][bp] = wave_sum(acc[r][q][bp]);
    const int r = lane % R, bp = lane / R;
    if (bp < BG && b0 + bp < B && rbase + r < a.Nrows) {
      float v0 = 0.f, v1 = 0.f;
#pragma unroll
      for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int pp = 0; pp < BG; ++pp)
          if (rr == r && pp == bp) {
            v0 = acc[rr][0][pp];
            v1 = acc[rr][NW - 1][pp];
          }
      float out;
      if (SW) {
        out = Elem<T>::round(Elem<T>::round(silu(Elem<T>::round(v0))) * Elem<T>::round(v1));
      } else {
        out = Elem<T>::round(v0);
        if (has_resid) out = Elem<T>::round(out + Raw<T>::f(rc));
      }
      int s = 0, loc = 0;
#pragma unroll
      for (int rr = 0; rr < R; ++rr)
        if (rr == r) {
          s = segi[rr];
          loc = local[rr];
        }
      Elem<T>::store(out_ptr<T>(a, s, b0 + bp, t, loc), out);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Batched decode GEMV on the matrix cores (bf16, 2 <= B <= 16). out[b, n] = W[n] . h[b] for a batch
// of up to 16 rows is a skinny GEMM whose batch dimension is exactly the 16 rows of
// v_mfma_f32_16x16x32_bf16: A = the (normalised) activation rows -- loaded per lane straight from
// memory (DX, rows in place), or for gathered rows staged in LDS (rows padded to K*2 + 16 bytes:
// conflict-free 16-byte reads); rows past B are zero --, B = 16 weight rows straight
// from memory (lane (row n, k-group g) holds 16 bytes of W[n]), and the C fragment already holds
// one output row per lane column and four batch rows per lane -- no cross-lane reduction, where the
// batched CUDA-style kernel above reduces every (row, batch row) dot product across a wave. A
// workgroup owns one 16-row output tile (two for SwiGLU: gate and up) and splits K over KSPLIT
// waves (4..16, so a launch keeps ~1000+ waves streaming weights); their partial tiles are summed
// through LDS by wave 0, which applies the same epilogues and rounding points as the kernels above.
// Requests: the activation rows first (small, from L2), then every weight fragment of the wave,
// then the waits. With rows in place (DX) no row is staged: each lane loads its own A fragments
// (batch row r, the wave's k-steps) straight from memory next to its weight fragments. Without an
// RMSNorm prologue the k-steps then wait for those loads only -- no LDS round trip and no barrier
// before the matrix-core steps, and the same sums as the staged form. With one, each lane also
// loads the norm weight's fragments; the row's sum of squares is the lane's fragment sums, summed
// over the row's four lanes (shuffles) and over the waves (16 floats per wave through LDS, one
// barrier), and each fragment is scaled in registers: round(x * rsqrt(ss / K + eps) * w), the
// staged form's formula (its sum of squares runs in another order).
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short mf_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float mf_f32x4;

// one staged 16-byte chunk c of a row scaled in place by the row's rsqrt and the norm weight
__device__ __forceinline__ void norm_chunk(unsigned char* row, int c, float rs, uint4 graw) {
  float xf[8], gw[8];
  Vec<bf16_t>::unpack(*reinterpret_cast<const uint4*>(row + c * 16), xf);
  Vec<bf16_t>::unpack(graw, gw);
#pragma unroll
  for (int e = 0; e < 8; ++e) xf[e] = Elem<bf16_t>::round(xf[e] * rs * gw[e]);
  *reinterpret_cast<uint4*>(row + c * 16) = Vec<bf16_t>::pack(xf);
}

template <int KSPLIT, int TPW, int KSW, bool SW, bool GA, bool HALF, bool DX>
__global__ __launch_bounds__(64 * KSPLIT * TPW) void decode_gemv_mfma_kernel(GemvArgs a, int steps_per_wave) {
  static_assert(!(DX && GA), "direct fragments read rows in place");
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = 64 * KSPLIT * TPW;               // TPW 16-row tiles per workgroup share the staging
  constexpr int NW = SW ? 2 : 1;
  constexpr int XC = 8;                                // staged 16-byte chunks per thread (host: 2K <= XC*NT)
  const int lane = threadIdx.x & 63, wwave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = wwave / KSPLIT, wave = wwave % KSPLIT;   // this wave's tile and K slice
  const int r = lane & 15, g = lane >> 4;
  const int K = a.K, B = a.B;
  const int kc = K / 8;                                // 16-byte chunks per row
  const int rowb = K * 2 + 16;                         // padded LDS row (bytes)
  unsigned char* hs = smem;                            // [16][rowb] staged rows (not with DX)
  float* red = reinterpret_cast<float*>(smem + (DX ? 0 : 16 * rowb));   // [TPW][KSPLIT][NW][64][4] partial tiles
  // tiles of tr real rows (16, or 8 for outputs with few tiles: twice the workgroups stream the
  // weights; lanes r >= 8 then read nothing and their output columns are dropped)
  constexpr int trs = HALF ? 3 : 4;                   // log2 of the real rows per tile (a compile-time
  constexpr int tr = 1 << trs;                         // choice: read from the arguments it cost a wait)
  const int n0 = min((int)(blockIdx.x * TPW + tile) << trs, ((a.Nrows - 1) >> trs) << trs);   // past the end: last tile
  const bool tile_live = ((int)(blockIdx.x * TPW + tile) << trs) < a.Nrows;
  const RowSeg seg0 = SW ? RowSeg{0, n0} : row_segment(a, n0);
  // a partial last tile (one segment only) reads its last real row in place of the missing ones
  const bool row_ok = r < tr && n0 + r < a.Nrows;
  const int wrow = seg0.local + (row_ok ? r : a.Nrows - 1 - n0);
  // this tile's weight rows (segment rows seg0.local .. +15; a lane reads row wrow)
  const bf16_t* wt0 = (const bf16_t*)pick_seg(seg0.s, a.seg[0].W, a.seg[1].W, a.seg[2].W) + (int64_t)seg0.local * K;
  const bf16_t* wt1 = SW ? (const bf16_t*)a.seg[1].W + (int64_t)seg0.local * K : wt0;

  // ---- requests: activation chunks (chunk i = row i / kc, column i % kc), the norm weight, this
  // wave's weight fragments, the residual operands -- in that order, then the waits. Rows in place
  // (GA false) take raw buffer loads: an offset past the resource reads zeros and makes no memory
  // request, so every load is issued unconditionally and the compiler can wait for the activation
  // rows alone before staging them, for the norm weight alone before the normalisation. (A load
  // that a lane predicate or branch may skip after them makes it wait for every load, the weight
  // burst included, before the staging: ~1-2 us of exposed weight latency per launch.)
  constexpr uint32_t kOOB = 0x80000000u;               // past every resource below (each < 2 GB)
  constexpr int GC = 4;                                // K <= 64 * GC * 8 (larger K loads in the loop)
  const bool g_early = a.g != nullptr && kc <= 64 * GC;
  const int nsteps = K / 32;
  const int s0 = wave * steps_per_wave;
  const int my_steps = min(steps_per_wave, nsteps - s0);
  const int wr = wrow - seg0.local;                    // 0..15
  uint4 xs[XC], gv[GC], wf[NW][KSW], xd[KSW], gd[KSW];
  uint32_t rres[4] = {0u, 0u, 0u, 0u};
  if constexpr (!GA) {
    const __amdgpu_buffer_rsrc_t rx =
        buf_rsrc(a.x, a.frag_in ? (uint32_t)(K * 32) : (uint32_t)(((int64_t)(B - 1) * a.x_bstride + K) * 2));
    if constexpr (DX) {
      // this lane's A fragments: batch row r (zeros past B), 16 bytes of each of the wave's k-steps
      // (in fragment order: chunk (s * 64 + lane), so a wave's request is one contiguous 1 KB)
#pragma unroll
      for (int j = 0; j < KSW; ++j) {
        const uint32_t off = j < my_steps && r < B
                                 ? (a.frag_in ? (uint32_t)(((s0 + j) * 64 + lane) * 16)
                                              : (uint32_t)(((int64_t)r * a.x_bstride + (s0 + j) * 32 + 8 * g) * 2))
                                 : kOOB;
        xd[j] = bld16(rx, off);
      }
      // the norm weight's fragments of the same k-steps (no norm: an empty resource, no requests)
      const __amdgpu_buffer_rsrc_t rgd = buf_rsrc(a.g, a.g != nullptr ? (uint32_t)(K * 2) : 0u);
#pragma unroll
      for (int j = 0; j < KSW; ++j)
        gd[j] = bld16(rgd, j < my_steps ? (uint32_t)(((s0 + j) * 32 + 8 * g) * 2) : kOOB);
    } else {
      // (whole slots past the rows are skipped by a uniform branch: the loads issued after every
      // activation slot do not depend on it, so the waits stay exact)
#pragma unroll
      for (int j = 0; j < XC; ++j) {
        xs[j] = make_uint4(0u, 0u, 0u, 0u);
        if (j * NT < B * kc) {                         // uniform
          const int i = threadIdx.x + j * NT;
          const uint32_t off = i < B * kc ? (uint32_t)(((int64_t)(i / kc) * a.x_bstride + (i % kc) * 8) * 2) : kOOB;
          xs[j] = bld16(rx, off);
        }
      }
    }
    if constexpr (!DX) {
      const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.g, g_early ? (uint32_t)(K * 2) : 0u);
#pragma unroll
      for (int i = 0; i < GC; ++i) gv[i] = bld16(rg, (uint32_t)(lane + 64 * i) * 16u);   // past K: zeros
    }
    const uint32_t wbytes = (uint32_t)(16 * K * 2);
    const __amdgpu_buffer_rsrc_t rw0 = buf_rsrc(wt0, wbytes);
    const __amdgpu_buffer_rsrc_t rw1 = buf_rsrc(wt1, wbytes);
#pragma unroll
    for (int j = 0; j < KSW; ++j) {
      const uint32_t off = j < my_steps && r < tr ? (uint32_t)((wr * K + (s0 + j) * 32 + 8 * g) * 2) : kOOB;
      wf[0][j] = bld16w(rw0, off);
      if (SW) wf[NW - 1][j] = bld16w(rw1, off);
    }
    if (!SW) {
      // the residual operands of this lane's outputs (row n0 + r, batch rows 4g + i), requested now so
      // the epilogue does not wait a memory round trip (wave 0 only: the other waves' resource is
      // empty; a branch here would make the compiler wait for these loads to merge the values)
      const uint32_t rbytes = a.resid != nullptr && wave == 0
                                  ? (uint32_t)(((int64_t)(B - 1) * a.resid_bstride + seg0.local + 16) * 2) : 0u;
      const __amdgpu_buffer_rsrc_t rr = buf_rsrc(a.resid, rbytes);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = min(4 * g + i, B - 1);
        rres[i] = bld2(rr, (uint32_t)(((int64_t)b * a.resid_bstride + seg0.local + (row_ok ? r : 0)) * 2));
      }
    }
  } else {
    // gathered rows (the first layer reads embedding rows by token id): predicated global loads
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int i = threadIdx.x + j * NT;
      xs[j] = make_uint4(0u, 0u, 0u, 0u);
      if (i < B * kc) {
        const int b = i / kc;
        const int64_t xrow = a.x_rows ? load_uniform(a.x_rows + b) : (int64_t)b;
        xs[j] = ld16((const bf16_t*)a.x + xrow * a.x_bstride + (int64_t)(i % kc) * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < GC; ++i) {
      gv[i] = make_uint4(0u, 0u, 0u, 0u);
      if (g_early && lane + 64 * i < kc) gv[i] = ld16((const bf16_t*)a.g + (lane + 64 * i) * 8);
    }
#pragma unroll
    for (int j = 0; j < KSW; ++j) {
      if (j < my_steps) {
        wf[0][j] = ldw16(wt0 + (int64_t)wr * K + (s0 + j) * 32 + 8 * g);
        if (SW) wf[NW - 1][j] = ldw16(wt1 + (int64_t)wr * K + (s0 + j) * 32 + 8 * g);
      }
    }
    if (!SW && a.resid && wave == 0) {                // uniform
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = min(4 * g + i, B - 1);
        const int64_t rrow = a.resid_rows ? a.resid_rows[b] : (int64_t)b;
        rres[i] = Raw<bf16_t>::load((const bf16_t*)a.resid + rrow * a.resid_bstride + seg0.local + (row_ok ? r : 0));
      }
    }
  }
  const int64_t t = a.uses_t ? load_uniform(a.t_dev) : 0;
  DH_ISSUE_FENCE();

  // ---- stage the rows (zeros past B), then normalise each once (wave w: rows w, w + KSPLIT, ...)
  if constexpr (!DX) {
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < 16 * kc) {
      const int b = i / kc;
      *reinterpret_cast<uint4*>(hs + b * rowb + (i % kc) * 16) = b < B ? xs[j] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  __syncthreads();
  }
  if (!DX && a.g != nullptr) {                         // uniform
    for (int b = wwave; b < B; b += KSPLIT * TPW) {
      float ss = 0.f;
      for (int c = lane; c < kc; c += 64) {
        float xf[8];
        Vec<bf16_t>::unpack(*reinterpret_cast<const uint4*>(hs + b * rowb + c * 16), xf);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += xf[e] * xf[e];
      }
      const float rs = rsqrtf(wave_sum(ss) / (float)K + a.eps);
      unsigned char* row = hs + b * rowb;
      if (g_early) {                                   // uniform
#pragma unroll
        for (int i = 0; i < GC; ++i)
          if (lane + 64 * i < kc) norm_chunk(row, lane + 64 * i, rs, gv[i]);
      } else {
        for (int c = lane; c < kc; c += 64) norm_chunk(row, c, rs, ld16((const bf16_t*)a.g + c * 8));
      }
    }
    __syncthreads();
  }

  // ---- DX with a norm: the rows' sums of squares (lane -> row's four lanes -> waves), then rsqrt
  float rsd = 1.f;
  const bool dnorm = DX && a.g != nullptr;
  if (dnorm) {                                         // uniform
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < KSW; ++j) {
      float xf[8];
      Vec<bf16_t>::unpack(xd[j], xf);                  // past the wave's steps: zeros
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += xf[e] * xf[e];
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    float* ssx = red + TPW * KSPLIT * NW * 64 * 4;     // [TPW * KSPLIT][16]
    if (g == 0) ssx[wwave * 16 + r] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < KSPLIT; ++w2) tot += ssx[(tile * KSPLIT + w2) * 16 + r];
    rsd = rsqrtf(tot / (float)K + a.eps);
  }

  // ---- this wave's k-steps on the matrix cores
  mf_f32x4 acc[NW];
#pragma unroll
  for (int q = 0; q < NW; ++q) acc[q] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KSW; ++j) {
    if (j < my_steps) {                                // uniform
      mf_bf16x8 av, bv;
      uint4 xa = DX ? xd[j] : *reinterpret_cast<const uint4*>(hs + r * rowb + ((s0 + j) * 32 + 8 * g) * 2);
      if (dnorm) {                                     // uniform
        float xf[8], gw[8];
        Vec<bf16_t>::unpack(xa, xf);
        Vec<bf16_t>::unpack(gd[j], gw);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = Elem<bf16_t>::round(xf[e] * rsd * gw[e]);
        xa = Vec<bf16_t>::pack(xf);
      }
      __builtin_memcpy(&av, &xa, 16);
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        __builtin_memcpy(&bv, &wf[q][j], 16);
        acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[q], 0, 0, 0);
      }
    }
  }
  // ---- partial tiles through LDS; wave 0 sums them and writes (row n0 + r, batch rows 4g + i)
#pragma unroll
  for (int q = 0; q < NW; ++q)
    *reinterpret_cast<mf_f32x4*>(red + (((tile * KSPLIT + wave) * NW + q) * 64 + lane) * 4) = acc[q];
  __syncthreads();
  if (wave == 0 && tile_live) {
    float v[NW][4];
#pragma unroll
    for (int q = 0; q < NW; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[q][i] = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < KSPLIT; ++w2)
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        const mf_f32x4 p = *reinterpret_cast<const mf_f32x4*>(red + (((tile * KSPLIT + w2) * NW + q) * 64 + lane) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[q][i] += p[i];
      }
    const int loc = seg0.local + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * g + i;
      if (b >= B || !row_ok) continue;
      float out;
      if (SW) {
        out = Elem<bf16_t>::round(Elem<bf16_t>::round(silu(Elem<bf16_t>::round(v[0][i]))) *
                                  Elem<bf16_t>::round(v[NW - 1][i]));
      } else {
        out = Elem<bf16_t>::round(v[0][i]);
        if (a.resid) out = Elem<bf16_t>::round(out + Raw<bf16_t>::f(rres[i]));
      }
      if (a.frag_out)                                  // fragment order (one segment, no t_stride)
        ((bf16_t*)a.seg[0].out)[((((int64_t)(loc >> 5) * 64 + ((loc >> 3) & 3) * 16 + b)) << 3) + (loc & 7)] =
            f32_to_bf16(out);
      else
        Elem<bf16_t>::store(out_ptr<bf16_t>(a, seg0.s, b, t, loc), out);
    }
  }
  advance_position(a);
}

// Many 16-row tiles without a residual (the vocabulary head at batch > 1): persistent workgroups,
// as many as the GPU has CUs, walk the groups of TPW tiles gridDim.x apart. The activation rows are
// staged and normalised once per workgroup instead of once per group, and each group's weights are
// requested before the previous group's matrix-core steps, so the weight stream does not stop at a
// group boundary. Per output element the arithmetic is the kernel above's.
// Every request is straight-line: the activation rows and the norm weight through raw buffer loads
// (past the rows: zeros, no memory request), and with FULL (every wave owns exactly KSW k-steps:
// K = 32 * KSPLIT * KSW) the weight loads and the k-steps without a predicate, and the next group's
// weights requested unconditionally (past the last group: the clamped last tile, loaded and unused).
// A predicated request makes the compiler wait for every load before the first use of any, which
// here meant waiting for the NEXT group's weights before each group's k-steps (measured: the
// batch-16 vocabulary head streamed at ~3 TB/s).
template <int KSPLIT, int TPW, int KSW, bool FULL>
__global__ __launch_bounds__(64 * KSPLIT * TPW) void decode_gemv_mfma_pers_kernel(GemvArgs a, int steps_per_wave,
                                                                                  int ngroups) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = 64 * KSPLIT * TPW;
  constexpr int XC = 8;                                // staged 16-byte chunks per thread (host: 2K <= XC*NT)
  constexpr uint32_t kOOB = 0x80000000u;               // past every resource below (each < 2 GB)
  const int lane = threadIdx.x & 63, wwave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = wwave / KSPLIT, wave = wwave % KSPLIT;
  const int r = lane & 15, g = lane >> 4;
  const int K = a.K, B = a.B;
  const int kc = K / 8;
  const int rowb = K * 2 + 16;
  unsigned char* hs = smem;                            // [16][rowb] staged rows
  float* red = reinterpret_cast<float*>(smem + 16 * rowb);   // [TPW][KSPLIT][64][4] partial tiles

  // rows in place (the host launches this kernel only without gathered rows)
  uint4 xs[XC];
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, (uint32_t)(((int64_t)(B - 1) * a.x_bstride + K) * 2));
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int i = threadIdx.x + j * NT;
    const uint32_t off = i < B * kc ? (uint32_t)(((int64_t)(i / kc) * a.x_bstride + (i % kc) * 8) * 2) : kOOB;
    xs[j] = bld16(rx, off);
  }
  constexpr int GC = 4;
  // FULL: K = 32 * KSPLIT * KSW <= 1024, so the norm weight always fits the early registers
  const bool g_early = a.g != nullptr && (FULL || kc <= 64 * GC);
  uint4 gv[GC];
  const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.g, g_early ? (uint32_t)(K * 2) : 0u);
#pragma unroll
  for (int i = 0; i < GC; ++i) gv[i] = bld16(rg, (uint32_t)(lane + 64 * i) * 16u);   // past K: zeros
  const int nsteps = K / 32;
  const int s0 = wave * steps_per_wave;
  const int my_steps = FULL ? KSW : min(steps_per_wave, nsteps - s0);
  // a group's tile geometry for this wave: first row, real rows, the tile's first weight row and the
  // row this lane reads within it; `valid`: the group exists (a request past the last one reads nothing)
  struct Geo { int n0, loc, s, wr; bool live, row_ok, valid; const bf16_t* wt; };
  auto geo = [&](int grp) {
    Geo q;
    const int tl = grp * TPW + tile;
    q.valid = grp < ngroups;
    q.n0 = min(tl * 16, ((a.Nrows - 1) / 16) * 16);
    q.live = tl * 16 < a.Nrows;
    const RowSeg sg = row_segment(a, q.n0);
    q.s = sg.s;
    q.row_ok = q.n0 + r < a.Nrows;
    q.loc = sg.local + r;
    q.wr = q.row_ok ? r : a.Nrows - 1 - q.n0;
    q.wt = (const bf16_t*)pick_seg(sg.s, a.seg[0].W, a.seg[1].W, a.seg[2].W) + (int64_t)sg.local * K;
    return q;
  };
  auto load_w = [&](uint4 (&wf)[KSW], const Geo& q) {
    if constexpr (FULL) {
      const __amdgpu_buffer_rsrc_t rw = buf_rsrc(q.wt, (uint32_t)(16 * K * 2));
#pragma unroll
      for (int j = 0; j < KSW; ++j)
        // ordinary loads (not bld16w's non-temporal ones): part of the head's rows then survives in the
        // memory-side cache until the next step's head (batch 16: 0.652 -> 0.650 ms per step)
        wf[j] = bld16(rw, q.valid ? (uint32_t)((q.wr * K + (s0 + j) * 32 + 8 * g) * 2) : kOOB);
    } else {
#pragma unroll
      for (int j = 0; j < KSW; ++j)
        if (j < my_steps) wf[j] = ld16(q.wt + (int64_t)q.wr * K + (s0 + j) * 32 + 8 * g);
    }
  };
  uint4 wa[KSW], wb[KSW];
  Geo ga = geo(blockIdx.x);
  load_w(wa, ga);
  const int64_t t = a.uses_t ? load_uniform(a.t_dev) : 0;
  DH_ISSUE_FENCE();

  // ---- stage the rows (zeros past B), then normalise each once (wave w: rows w, w + KSPLIT * TPW, ...)
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < 16 * kc) {
      const int b = i / kc;
      *reinterpret_cast<uint4*>(hs + b * rowb + (i % kc) * 16) = b < B ? xs[j] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  __syncthreads();
  if (a.g != nullptr) {                                // uniform
    for (int b = wwave; b < B; b += KSPLIT * TPW) {
      float ss = 0.f;
      for (int c = lane; c < kc; c += 64) {
        float xf[8];
        Vec<bf16_t>::unpack(*reinterpret_cast<const uint4*>(hs + b * rowb + c * 16), xf);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += xf[e] * xf[e];
      }
      const float rs = rsqrtf(wave_sum(ss) / (float)K + a.eps);
      unsigned char* row = hs + b * rowb;
      if (FULL || g_early) {                           // uniform
#pragma unroll
        for (int i = 0; i < GC; ++i)
          if (lane + 64 * i < kc) norm_chunk(row, lane + 64 * i, rs, gv[i]);
      } else {
        for (int c = lane; c < kc; c += 64) norm_chunk(row, c, rs, ld16((const bf16_t*)a.g + c * 8));
      }
    }
    __syncthreads();
  }

  // ---- one group: the next group's weights requested first, then this group's k-steps, partial
  // tiles through LDS, wave 0 of each tile sums them and writes (row n0 + r, batch rows 4g + i).
  // With FULL every wave of the tile sums them and the stores go through a buffer resource whose
  // offsets drop the other waves' and the dead outputs' stores: no branch around a memory request.
  auto group = [&](int grp, const Geo& q, const uint4 (&wf)[KSW], uint4 (&wn)[KSW], Geo& qn) {
    const int nxt = grp + (int)gridDim.x;
    if (FULL || nxt < ngroups) {                       // FULL: unconditional (past the last group: no request)
      qn = geo(nxt);
      load_w(wn, qn);
    }
    mf_f32x4 acc = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KSW; ++j) {
      if (FULL || j < my_steps) {                      // uniform
        mf_bf16x8 av, bv;
        const uint4 xa = *reinterpret_cast<const uint4*>(hs + r * rowb + ((s0 + j) * 32 + 8 * g) * 2);
        __builtin_memcpy(&av, &xa, 16);
        __builtin_memcpy(&bv, &wf[j], 16);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
      }
    }
    *reinterpret_cast<mf_f32x4*>(red + ((tile * KSPLIT + wave) * 64 + lane) * 4) = acc;
    __syncthreads();
    if constexpr (FULL) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w2 = 0; w2 < KSPLIT; ++w2) {
        const mf_f32x4 p = *reinterpret_cast<const mf_f32x4*>(red + ((tile * KSPLIT + w2) * 64 + lane) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += p[i];
      }
      bf16_t* ob = (bf16_t*)pick_seg(q.s, a.seg[0].out, a.seg[1].out, a.seg[2].out) +
                   t * pick_seg(q.s, a.seg[0].t_stride, a.seg[1].t_stride, a.seg[2].t_stride);
      const int64_t bs = pick_seg(q.s, a.seg[0].out_bstride, a.seg[1].out_bstride, a.seg[2].out_bstride);
      const int ns = pick_seg(q.s, a.seg[0].N, a.seg[1].N, a.seg[2].N);
      const __amdgpu_buffer_rsrc_t ro = buf_rsrc(ob, (uint32_t)(((int64_t)(B - 1) * bs + ns) * 2));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;
        const bool st = wave == 0 && q.live && b < B && q.row_ok;
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f32_to_bf16(v[i]), ro,
                                              st ? (uint32_t)(((int64_t)b * bs + q.loc) * 2) : kOOB, 0, 0);
      }
    } else if (wave == 0 && q.live) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w2 = 0; w2 < KSPLIT; ++w2) {
        const mf_f32x4 p = *reinterpret_cast<const mf_f32x4*>(red + ((tile * KSPLIT + w2) * 64 + lane) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += p[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;
        if (b >= B || !q.row_ok) continue;
        Elem<bf16_t>::store(out_ptr<bf16_t>(a, q.s, b, t, q.loc), Elem<bf16_t>::round(v[i]));
      }
    }
    __syncthreads();                                   // red is rewritten by the next group
  };
  Geo gb = ga;
  for (int grp = blockIdx.x; grp < ngroups;) {
    group(grp, ga, wa, wb, gb);
    grp += gridDim.x;
    if (grp >= ngroups) break;
    group(grp, gb, wb, wa, ga);
    grp += gridDim.x;
  }
  advance_position(a);
}

template <int KSPLIT, int TPW, int KSW, bool SW>
void launch_mfma_k(const GemvArgs& a, int steps_per_wave, hipStream_t s) {
  const bool dx = !a.x_rows && !a.resid_rows;         // rows in place: no staging (see the kernel)
  const size_t lds = (dx ? (size_t)TPW * KSPLIT * 16 * 4 : (size_t)16 * (a.K * 2 + 16)) +
                     (size_t)TPW * KSPLIT * (SW ? 2 : 1) * 64 * 16;
  auto kern = a.x_rows || a.resid_rows ? &decode_gemv_mfma_kernel<KSPLIT, TPW, KSW, SW, true, false, false>
                                       : &decode_gemv_mfma_kernel<KSPLIT, TPW, KSW, SW, false, false, false>;
  if (dx) kern = &decode_gemv_mfma_kernel<KSPLIT, TPW, KSW, SW, false, false, true>;
  if constexpr (!SW && TPW == 1)
    if (a.tile_rows == 8)
      kern = dx ? &decode_gemv_mfma_kernel<KSPLIT, TPW, KSW, SW, false, true, true>
                : &decode_gemv_mfma_kernel<KSPLIT, TPW, KSW, SW, false, true, false>;
  if (lds > 64 * 1024)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
  const int tiles = (a.Nrows + a.tile_rows - 1) / a.tile_rows;
  kern<<<dim3((tiles + TPW - 1) / TPW), dim3(64 * KSPLIT * TPW), lds, s>>>(a, steps_per_wave);
}

// K split: enough waves to stream the weights (~1024+ per launch), at least 4 per workgroup (they
// share the staged rows) and enough for the staging (2K <= 8 * 64 * KSPLIT). The normalised
// launches keep it without staging too: measured at batch 16, 4 or 16 waves per workgroup instead
// of 8 made the decode step 1-3% slower.
// (SwiGLU: at most 8 waves -- two weight tiles per wave do not fit 16 waves' registers)
bool mfma_gemv_fits(const GemvArgs& a, bool swiglu) {
  if (a.B < 2 || a.B > 16 || a.K % 32 != 0 || a.K > (swiglu ? 2048 : 4096)) return false;
  // rows in place are read through buffer resources of < 2 GB (activations, residual)
  const int64_t lim = (int64_t)1 << 30;                // elements of 2 bytes
  if ((int64_t)(a.B - 1) * a.x_bstride + a.K >= lim) return false;
  if (a.resid && (int64_t)(a.B - 1) * a.resid_bstride + a.Nrows >= lim) return false;
  if (a.nseg == 1 && !swiglu) return true;            // a partial last tile is handled
  for (int s = 0; s < a.nseg; ++s)
    if (a.seg[s].N % 16 != 0) return false;
  return true;
}

template <bool SW>
void launch_mfma(const GemvArgs& a0, hipStream_t s) {
  // outputs of fewer than 128 sixteen-row tiles (the 1024-row projections) run tiles of 8 real rows:
  // twice the workgroups streaming the weights (rows in place only)
  GemvArgs a = a0;
  if (!SW && a.nseg == 1 && !a.x_rows && !a.resid_rows && (a.Nrows + 15) / 16 < 128) a.tile_rows = 8;
  const int tiles = (a.Nrows + a.tile_rows - 1) / a.tile_rows, nsteps = a.K / 32;
  constexpr int kmax = SW ? 8 : 16;
  int ks = 4;
  while (ks < kmax && (tiles * ks < 1024 || a.K > 256 * ks)) ks *= 2;
  const int spw = (nsteps + ks - 1) / ks;             // <= 8: K <= 256 * ks
  const bool small = spw <= 4;
  if constexpr (!SW) {
    // many tiles (the vocabulary head): four tiles per workgroup share one staging of the rows; with
    // no residual, persistent workgroups walk the tile groups
    if (ks == 4 && tiles >= 4 * 512) {
      if (a.resid == nullptr && a.x_rows == nullptr) {
        const int ngroups = (tiles + 3) / 4;
        int dev = 0, ncu = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
          ncu = 256;
        const int grid = ngroups < ncu ? ngroups : ncu;
        const size_t lds = (size_t)16 * (a.K * 2 + 16) + (size_t)4 * 4 * 64 * 16;
        auto go = [&](auto kern) {
          if (lds > 64 * 1024)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
          kern<<<dim3(grid), dim3(1024), lds, s>>>(a, spw, ngroups);
        };
        const bool full = nsteps == 4 * (small ? 4 : 8);   // every wave exactly KSW k-steps
        if (small) {
          if (full) go(&decode_gemv_mfma_pers_kernel<4, 4, 4, true>); else go(&decode_gemv_mfma_pers_kernel<4, 4, 4, false>);
        } else {
          if (full) go(&decode_gemv_mfma_pers_kernel<4, 4, 8, true>); else go(&decode_gemv_mfma_pers_kernel<4, 4, 8, false>);
        }
        return;
      }
      if (small) launch_mfma_k<4, 4, 4, SW>(a, spw, s); else launch_mfma_k<4, 4, 8, SW>(a, spw, s);
      return;
    }
  }
  if constexpr (!SW) {
    // rows in place without a norm (no staging: each wave loads its own A fragments): fewer, longer
    // waves -- the fewest (at least 4) whose k-steps fit 12 per wave. Measured at batch 16: the
    // 1024 x 2816 down projection 7.36 -> 6.53 us per launch with 8 waves of 11 k-steps instead of
    // 16 of 6 (4 waves of 22: 7.0 us); the staged, normalised launches lose with fewer waves.
    if (a.g == nullptr && !a.x_rows && !a.resid_rows) {
      int k2 = 4;
      while (k2 < 16 && nsteps > 12 * k2) k2 *= 2;
      const int sp = (nsteps + k2 - 1) / k2;           // <= 8 at k2 = 16 (K <= 4096)
      if (k2 == 4) {
        if (sp <= 4) launch_mfma_k<4, 1, 4, SW>(a, sp, s);
        else if (sp <= 8) launch_mfma_k<4, 1, 8, SW>(a, sp, s);
        else launch_mfma_k<4, 1, 12, SW>(a, sp, s);
      } else if (k2 == 8) {
        if (sp <= 8) launch_mfma_k<8, 1, 8, SW>(a, sp, s); else launch_mfma_k<8, 1, 12, SW>(a, sp, s);
      } else {
        if (sp <= 4) launch_mfma_k<16, 1, 4, SW>(a, sp, s); else launch_mfma_k<16, 1, 8, SW>(a, sp, s);
      }
      return;
    }
  }
  if (ks == 4) { if (small) launch_mfma_k<4, 1, 4, SW>(a, spw, s); else launch_mfma_k<4, 1, 8, SW>(a, spw, s); }
  else if (ks == 8) { if (small) launch_mfma_k<8, 1, 4, SW>(a, spw, s); else launch_mfma_k<8, 1, 8, SW>(a, spw, s); }
  else if constexpr (!SW) {
    if (small) launch_mfma_k<16, 1, 4, SW>(a, spw, s); else launch_mfma_k<16, 1, 8, SW>(a, spw, s);
  }
}

constexpr int kStageBytes = 96 * 1024;                 // LDS for staged batch rows
#ifndef DH_GEMV_ROW_THREADS
#define DH_GEMV_ROW_THREADS 256
#endif
constexpr int kRowThreads = DH_GEMV_ROW_THREADS;      // workgroup of the single-row kernel

template <typename T, int R, int CG, bool SW>
void launch(const GemvArgs& a, hipStream_t s) {
  const int rows_per_block = kWaves * R;
  const int grid = (a.Nrows + rows_per_block - 1) / rows_per_block;
  const size_t stage = (size_t)a.B * a.K * sizeof(T);
  if (a.B > 1 && stage <= (size_t)kStageBytes) {
    if (stage > 64 * 1024)   // past the default dynamic LDS limit (gfx950 has 160 KB per CU)
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_gemv_staged_kernel<T, R, CG, SW>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kStageBytes);
    decode_gemv_staged_kernel<T, R, CG, SW><<<dim3(grid), dim3(kThreads), stage, s>>>(a);
    return;
  }
  if (a.B == 1) {
    constexpr int NT = kRowThreads;
    const int grid1 = (a.Nrows + (NT / 64) * R - 1) / ((NT / 64) * R);
    if (a.x_rows || a.resid_rows)
      decode_gemv_row_kernel<T, R, CG, SW, NT, true><<<dim3(grid1), dim3(NT), 0, s>>>(a);
    else
      decode_gemv_row_kernel<T, R, CG, SW, NT, false><<<dim3(grid1), dim3(NT), 0, s>>>(a);
    return;
  }
  // batch rows per pass: as many as the activation chunks' registers allow
  constexpr int BG = CG <= 2 ? 8 : (CG <= 6 ? 4 : 2);
  decode_gemv_kernel<T, R, CG, BG, SW><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
}

template <typename T, int CG, bool SW>
void pick_r(const GemvArgs& a, int R, hipStream_t s) {
  if constexpr (!SW) {
    if (R >= 4) {
      launch<T, 4, CG, SW>(a, s);
      return;
    }
  }
  if (R >= 2) launch<T, 2, CG, SW>(a, s);
  else launch<T, 1, CG, SW>(a, s);
}

template <typename T, bool SW>
void pick_cg(const GemvArgs& a, int C, int R, hipStream_t s) {
  if (C <= 2) pick_r<T, 2, SW>(a, R, s);
  else if (C <= 4) pick_r<T, 4, SW>(a, R, s);
  else if (C <= 6) pick_r<T, 6, SW>(a, R < 2 ? R : 2, s);
  else pick_r<T, 12, SW>(a, 1, s);
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

// Rows per wave. Single row (measured on MI355X, weights streamed from HBM): about 4 KB of weights
// per wave while the launch keeps >= ~1.5k waves -- two rows of K = 1024 bf16 for the 3072-row
// projection, one row for 1024-row outputs, for SwiGLU (whose wave already reads a gate and an up
// row) and for K = 2816; four rows for the vocabulary head (> 12k waves). Batched calls stage the
// rows once per workgroup and reuse each weight chunk across all of them, so more rows per wave
// pay off there.
int rows_per_wave(int B, int Nrows, int K, int esz, bool swiglu) {
  if (B == 1) return Nrows >= 16384 ? 4 : (!swiglu && K * esz <= 2048 && Nrows >= 3072 ? 2 : 1);
  return Nrows >= 2048 ? 4 : 2;
}

}  // namespace

extern "C" int64_t dh_decode_gemv_candidates(int dtype, int N, int K) {
  if ((dtype != DH_F32 && dtype != DH_BF16) || N < 1 || K < 1) return 0;
  const int R = rows_per_wave(1, N, K, dtype == DH_BF16 ? 2 : 4, false);
  const int rows_per_block = (kRowThreads / 64) * R;
  return (N + rows_per_block - 1) / rows_per_block;
}

extern "C" int dh_decode_gemv(int dtype, const void* x, int64_t x_bstride, const int64_t* x_rows,
                              const void* norm_w, float eps, int nseg, const void* const* W,
                              void* const* out, const int64_t* out_bstride, const int64_t* out_t_stride,
                              const int* N, const void* resid, int64_t resid_bstride,
                              const int64_t* resid_rows, int flags, const int64_t* t_dev, int64_t* t_advance,
                              void* argmax_cand, int B, int K, void* stream) {
  const char* who = "dh_decode_gemv";
  DH_REQUIRE(flags >= 0 && flags <= 7, DH_ERR_INVALID_ARG, "%s: flags %d", who, flags);
  const int swiglu = flags & DH_GEMV_SWIGLU;
  const bool frag_out = (flags & DH_GEMV_FRAG_OUT) != 0, frag_in = (flags & DH_GEMV_FRAG_IN) != 0;
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  const int vec = dtype == DH_BF16 ? 8 : 4;             // elements per 16-byte chunk
  DH_REQUIRE(B >= 1 && K >= vec && K % vec == 0, DH_ERR_UNSUPPORTED_SHAPE,
             "%s: B=%d K=%d (K must be a multiple of %d: rows are read in 16-byte chunks)", who, B, K, vec);
  DH_REQUIRE(nseg >= 1 && nseg <= kMaxSeg, DH_ERR_INVALID_ARG, "%s: nseg=%d not in [1,%d]", who, nseg, kMaxSeg);
  DH_REQUIRE(!swiglu || nseg == 2, DH_ERR_INVALID_ARG, "%s: SwiGLU needs exactly the gate and up segments", who);
  DH_REQUIRE(!swiglu || !resid, DH_ERR_INVALID_ARG, "%s: SwiGLU and residual cannot be combined", who);
  DH_REQUIRE(!resid || nseg == 1, DH_ERR_INVALID_ARG, "%s: a residual needs a single segment", who);
  DH_REQUIRE(x && W && out && out_bstride && out_t_stride && N && t_dev, DH_ERR_INVALID_ARG, "%s: null pointer argument",
             who);
  DH_REQUIRE(aligned(x, 16) && (x_bstride * (dtype == DH_BF16 ? 2 : 4)) % 16 == 0 && (!norm_w || aligned(norm_w, 16)),
             DH_ERR_INVALID_ARG, "%s: x rows and the norm weight need 16-byte alignment", who);
  DH_REQUIRE(!argmax_cand || (B == 1 && nseg == 1 && !swiglu && !resid), DH_ERR_INVALID_ARG,
             "%s: argmax candidates need B = 1 and one plain output segment", who);
  GemvArgs a{};
  a.cand = (Cand*)argmax_cand;
  a.x = x;
  a.x_bstride = x_bstride;
  a.x_rows = x_rows;
  a.g = norm_w;
  a.eps = eps;
  a.resid = resid;
  a.resid_bstride = resid_bstride;
  a.resid_rows = resid_rows;
  a.t_dev = t_dev;
  a.t_advance = t_advance;
  a.nseg = nseg;
  a.B = B;
  a.K = K;
  int total = 0;
  for (int s = 0; s < nseg; ++s) {
    DH_REQUIRE(W[s] && out[s] && N[s] >= 1, DH_ERR_INVALID_ARG, "%s: segment %d incomplete", who, s);
    DH_REQUIRE(aligned(W[s], 16), DH_ERR_INVALID_ARG, "%s: segment %d weights need 16-byte alignment", who, s);
    a.seg[s] = Seg{W[s], out[s], out_bstride[s], out_t_stride[s], N[s]};
    a.uses_t |= out_t_stride[s] != 0;
    total += N[s];
  }
  DH_REQUIRE(!t_advance || !a.uses_t, DH_ERR_INVALID_ARG,
             "%s: a launch that advances the position cannot also address its outputs through it", who);
  if (swiglu) {
    DH_REQUIRE(N[0] == N[1], DH_ERR_INVALID_ARG, "%s: gate and up rows differ (%d, %d)", who, N[0], N[1]);
    total = N[0];
  }
  a.Nrows = total;
  a.tile_rows = 16;
  const int C = (K / vec + 63) / 64;
  DH_REQUIRE(C <= 12, DH_ERR_UNSUPPORTED_SHAPE, "%s: K=%d exceeds %d elements per row", who, K, 12 * 64 * vec);
  const int esz = dtype == DH_BF16 ? 2 : 4;
  const int R = rows_per_wave(B, a.Nrows, K, esz, swiglu != 0);
  hipStream_t s = (hipStream_t)stream;
  if (frag_out || frag_in) {
    // fragment order exists on the batched matrix-core path only, with the rows in place (the kernels
    // that read their activation fragments straight from memory), and not on the persistent
    // vocabulary-head form (many tiles without a residual), which stages its rows
    DH_REQUIRE(dtype == DH_BF16 && !argmax_cand && !x_rows && !resid_rows && mfma_gemv_fits(a, swiglu != 0) &&
                   (swiglu || resid || (a.Nrows + 15) / 16 < 4 * 512),
               DH_ERR_INVALID_ARG,
               "%s: fragment-ordered activations need the batched matrix-core path (bf16, 2 <= B <= 16, rows in place)",
               who);
    DH_REQUIRE(!frag_out || (swiglu && out_t_stride[0] == 0 && N[0] % 32 == 0), DH_ERR_INVALID_ARG,
               "%s: fragment-ordered outputs need a SwiGLU launch with N a multiple of 32 and no t_stride", who);
    DH_REQUIRE(!frag_in || (K % 32 == 0 && aligned(x, 16)), DH_ERR_INVALID_ARG,
               "%s: fragment-ordered activations need K a multiple of 32", who);
    a.frag_out = frag_out;
    a.frag_in = frag_in;
  }
  if (dtype == DH_BF16 && !argmax_cand && mfma_gemv_fits(a, swiglu != 0)) {
    if (swiglu) launch_mfma<true>(a, s); else launch_mfma<false>(a, s);
    return dh_check_launch(who);
  }
  if (dtype == DH_BF16) {
    if (swiglu) pick_cg<bf16_t, true>(a, C, R, s); else pick_cg<bf16_t, false>(a, C, R, s);
  } else {
    if (swiglu) pick_cg<float, true>(a, C, R, s); else pick_cg<float, false>(a, C, R, s);
  }
  return dh_check_launch(who);
}
