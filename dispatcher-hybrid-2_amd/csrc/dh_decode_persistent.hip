// One batch-1 bf16 decode step as a single persistent launch (dh_decode_persistent_step).
//
// The graphed decoder runs the step as ~94 dependent launches (reference dispatcher_hybrid/
// decoding.py:437-488 captures the same chain); each launch pays the graph node's ~1.6 us plus a
// cold start of its own weight stream. Here one workgroup per compute unit stays resident for the
// whole step and walks the same phases in the same order. A phase first requests everything it
// will read that no other workgroup of this launch writes (its weight rows, cached keys and
// values, ring values, the position-dependent history rows), then waits for its inputs, so the
// weight stream of a phase overlaps the hand-off of the previous one.
//
// Hand-off without fences or counters: every word a phase produces for another workgroup carries
// the producing phase's tag -- bf16 values as 32-bit words (value << 16 | 16-bit tag), fp32 values
// as 64-bit words (value | 32-bit tag << 32) -- written with agent-scope stores (write-through to
// memory) and read with agent-scope loads (never a stale cache line), and a consumer polls until
// every word it needs carries the tag it expects. A word is written whole, so a matching tag means
// a current value. Tags derive from an epoch the launch advances at its end, so words left from
// an earlier launch never match. Every wait is bounded (200 ms of wall clock, 4M polls); a timeout raises a
// flag every other wait observes, so all waves end and the step reports the failure.
//
// The arithmetic of each phase is that of the launch it replaces -- the single-row dh_decode_gemv
// kernel (RMSNorm over 256 threads, per-lane chunk sums, DPP wave sums, the same rounding points),
// dh_decode_gates' readout, dh_decode_scan_out's recurrence, the split decode attention and its
// combine, and dh_argmax_reduce's order -- so the logits and tokens equal the graphed step's bit
// for bit.
#include "dh_common.h"

namespace {

constexpr int kPT = 256;                 // threads per workgroup, as the single-row GEMV kernel
constexpr int kPW = kPT / 64;
constexpr int kLW = DH_PERSISTENT_LAYER_WORDS;
constexpr int kMaxLayers = 64;
constexpr int kLMax = 12;                // recurrence levels held in registers
constexpr int kSplitS = 16;              // attention window segments
constexpr int kHD = 64;                  // attention head width
constexpr int kRecW = 72;                // 64-bit words per segment record (m, l, kHD outputs): 64-byte multiple
static_assert(kRecW >= 2 + kHD && kRecW % 8 == 0, "segment records fill whole 64-byte segments");
constexpr int kUT = 128;                 // threads per attention segment unit (two per workgroup)
constexpr int kMaxSeg = DH_PERSISTENT_MAX_WINDOW / kSplitS;
constexpr uint64_t kSpinTicks = 20000000ull;   // 200 ms of the 100 MHz real-time counter
constexpr uint32_t kMaxPolls = 1u << 22;       // and at most this many polls per wait

// layer table fields
enum : int {
  F_KIND = 0, F_NORM1 = 1,
  // tree layer
  F_WIN = 2, F_WGH = 3, F_WGS = 4, F_WI = 5, F_WF = 6, F_WR = 7, F_BI = 8, F_BF = 9, F_BR = 10, F_WOUT = 11,
  F_BHIST = 12, F_RGHIST = 13, F_VRING = 14,
  // attention layer
  F_WQ = 2, F_WK = 3, F_WV = 4, F_WO = 5, F_KC = 6, F_VC = 7, F_COS = 8, F_SIN = 9, F_WINDOW = 10,
  // both
  F_NORM2 = 15, F_WGATE = 16, F_WUP = 17, F_WDOWN = 18,
};

// A layer's row of the layer table, read from the workgroup's LDS copy: LDS reads wait on the LDS
// counter only, so a table field read after a phase's wait never waits for the weight requests in
// flight (a table read through global memory would: vector-memory loads retire in order).
typedef const __attribute__((address_space(3))) int64_t lds_i64;
struct LayerRef {
  lds_i64* p;
  __device__ __forceinline__ int64_t operator[](int f) const { return p[f]; }
  __device__ __forceinline__ LayerRef next() const { return LayerRef{p + DH_PERSISTENT_LAYER_WORDS}; }
};

struct PArgs {
  const int64_t* table;      // device, n_layers * kLW words
  int n_layers;
  const bf16_t* emb;         // (V, d) embedding, also the vocabulary head
  const bf16_t* norm_out;
  int64_t* t_dev;
  int64_t* token;            // in: this step's token; out: the greedy pick
  int64_t* tok_hist;         // nullable: pick stored at tok_hist[t + 1] when below hist_len
  int64_t hist_len;
  bf16_t* logits;            // (V)
  int64_t* epoch;            // launches so far (tags)
  uint32_t* status;          // [0] abort flag, [1] first failing phase + 1
  uint32_t *xw, *i3w, *hw, *yw;   // tagged bf16 vectors: x, in-projection group, h, y
  int n3w, nhw;                    // padded extents (words) of i3w and hw
  uint64_t *coefw, *partw, *candw;                     // tagged fp32 records
  uint64_t* trace;           // nullable: per-phase timestamps (dh_decode_persistent_trace)
  float eps;
  int d, GH, H, hd, L, ff, V, Tmax, nph;
};

// ---- element helpers (bf16 only)
__device__ __forceinline__ void unpack8(const uint4& v, float (&o)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o[2 * j] = __uint_as_float(w[j] << 16);
    o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float (&o)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = (uint32_t)f32_to_bf16(o[2 * j]) | ((uint32_t)f32_to_bf16(o[2 * j + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ float rnd(float v) { return Elem<bf16_t>::round(v); }
__device__ __forceinline__ float bfv(uint32_t raw16) { return __uint_as_float(raw16 << 16); }
__device__ __forceinline__ float silu(float x) { return x * dh_sigmoid(x); }
// Global-memory access through the addresses in the layer table: those are generic pointers to the
// compiler (read from memory), which would make every access a flat one, counted against the LDS
// counter too, so each LDS wait would also wait for the weight fetches in flight. Rebuilding the
// pointer from its integer value in the global address space keeps them global loads and stores
// (a cast of the generic pointer itself is dropped).
typedef unsigned int gu32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int gu32x2 __attribute__((ext_vector_type(2)));
#define DH_GLOBAL(T, p) ((const __attribute__((address_space(1))) T*)(uintptr_t)(p))
#define DH_GLOBAL_W(T, p) ((__attribute__((address_space(1))) T*)(uintptr_t)(p))
__device__ __forceinline__ uint4 ld16(const void* p) {
  const gu32x4 v = *DH_GLOBAL(gu32x4, p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// weight rows, streamed once per step: non-temporal loads, so they do not push the step's state
// (ring slots, history rows, cached keys and values) out of L2
__device__ __forceinline__ uint4 ldw16(const void* p) {
  const gu32x4 v = __builtin_nontemporal_load(DH_GLOBAL(gu32x4, p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(const void* p) {
  const gu32x2 v = *DH_GLOBAL(gu32x2, p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ bf16_t ld2(const bf16_t* p) { return *DH_GLOBAL(bf16_t, p); }
__device__ __forceinline__ void st2(bf16_t* p, bf16_t v) { *DH_GLOBAL_W(bf16_t, p) = v; }
__device__ __forceinline__ void st8(void* p, uint2 v) {
  gu32x2 w;
  w.x = v.x;
  w.y = v.y;
  *DH_GLOBAL_W(gu32x2, p) = w;
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xb1, 0xf>(v));
  v = fmaxf(v, dpp_move<0x4e, 0xf>(v));
  v = fmaxf(v, dpp_move<0x141, 0xf>(v));
  v = fmaxf(v, dpp_move<0x140, 0xf>(v));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---- tags and tagged words
struct Tags {
  uint64_t base;             // epoch * nph
  __device__ __forceinline__ uint32_t t16(int ph) const { return (uint32_t)((base + (uint64_t)ph) % 65535ull) + 1u; }
  __device__ __forceinline__ uint32_t t32(int ph) const { return (uint32_t)((base + (uint64_t)ph) % 4294967295ull) + 1u; }
};
__device__ __forceinline__ void put16(uint32_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint32_t)f32_to_bf16(v) << 16) | tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put32(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t get16(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get32(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes of tagged words through the memory-side path (sc1: no stale L2 line)
__device__ __forceinline__ uint4 get16x4(const uint32_t* base, int nwords, int word) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(base), (short)0, nwords * 4, 0x00020000);
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)word * 4u, 0, 16));
}
__device__ __forceinline__ bool tag_ok(uint32_t w, uint32_t tag) { return (w & 0xffffu) == tag; }
// The x vector (the residual stream, written by one wave per row, the four rows of a workgroup
// consecutive) keeps each workgroup's four words in a 64-byte segment of its own: writers from
// several workgroups sharing a segment made every hand-off of x ~0.2 us slower (probe, 256
// workgroups). Word n of x sits at xpos(n); a 4-word chunk c at c * kXSeg.
constexpr int kXSeg = 16;
__device__ __forceinline__ int xpos(int n) { return (n >> 2) * kXSeg + (n & 3); }
static_assert(kPW == 4, "xpos: the four x rows of a workgroup share a segment");
// Likewise the phases of three rows per wave (the in-projection group V0 | A or q | k | v, and h):
// the kR3 rows of a workgroup in a 64-byte segment, row n at p3(n). The in-projection group is
// laid out by its global row (V0 then A; q, k, v), as its workgroups produce it.
constexpr int kR3 = 3 * kPW;
static_assert(kR3 <= kXSeg && kR3 % 4 == 0, "p3: a workgroup's rows fill one segment in whole chunks");
__device__ __forceinline__ int p3(int n) { return (n / kR3) * kXSeg + n % kR3; }
__host__ __device__ constexpr int p3_extent(int n) { return (n + kR3 - 1) / kR3 * kXSeg; }
__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

// Optional timing record of a traced step: per workgroup and phase, the 100 MHz real-time counter
// when the phase starts (k = 0), when its wait for other workgroups' words ended (k = 1; a phase
// without a wait in this workgroup leaves 0) and when it ends (k = 2). Thread 0 stamps.
#define DH_MARK(a, ph, k)                                                                             \
  do {                                                                                                \
    if ((a).trace && threadIdx.x == 0)                                                                \
      (a).trace[((int64_t)blockIdx.x * (a).nph + (ph)) * 3 + (k)] = now_ticks();                      \
  } while (0)

__device__ __forceinline__ bool aborted(const PArgs& a) { return get16(a.status) != 0u; }
// the first failure records its phase + 1, and in decimal digits above it the wait's end condition
// (thousands: 1 another wait failed, 2 time, 3 rounds) and its rounds (ten-thousands, capped)
__device__ __forceinline__ void raise_abort(const PArgs& a, int ph, uint32_t why = 0u, uint32_t polls = 0u) {
  if (__hip_atomic_fetch_add(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
    __hip_atomic_store(a.status + 1, (uint32_t)(ph + 1) + why * 1000u + (polls < 9999u ? polls : 9999u) * 10000u,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wait's end condition, evaluated from the status word loaded in the same batch as the polled
// data (a separate load would add a memory round trip to every round): another wait timed out,
// or this one has run 200 ms or kMaxPolls rounds.
struct Waiter {
  uint64_t t0;
  uint32_t polls, why;
  __device__ __forceinline__ Waiter() : t0(now_ticks()), polls(0), why(0) {}
  __device__ __forceinline__ bool expired(uint32_t status) {
    ++polls;
    why = status != 0u ? 1u : (now_ticks() - t0 > kSpinTicks ? 2u : (polls > kMaxPolls ? 3u : 0u));
    return why != 0u;
  }
};

// LDS of a workgroup. A phase may write, before its first barrier, only what the previous phase
// no longer reads after its last one: the RMSNorm weight has its own region (sg), written at the
// start of a phase while slower waves may still read the previous phase's staged row in sx.
struct Smem {
  uint4 sx[3072 / 8];            // staged activation row (chunks)
  uint4 sg[1024 / 8];            // RMSNorm weight (chunks)
  float red[kPW];
  int stop;                        // a wait's end condition, from thread 0 to the workgroup
  float2 coef[64 * kLMax];       // scan: {fg, ig * r_src} per (head, level)
  Cand wbest[kPW];
  // attention segment units (two per workgroup)
  float qs[2][kHD], ks[2][kHD], vsh[2][kHD];
  float sc[2][kMaxSeg];
  float ared[2][2];
  float part[2][2][kHD];
  // attention combine: the head's segment records, gathered by the workgroup's waves
  float cm[kSplitS], cl[kSplitS], co[kSplitS][kHD];
};

// Workgroup wait for n tagged bf16 words (n % 4 == 0, n <= 4 * kPT * 3; contiguous, or laid out by
// p3); the values land in dst (LDS) as bf16. One barrier per round: thread 0 publishes the end condition through LDS before it
// (a later round's write may race a slow thread's read of the earlier value; the condition only
// ever turns true). Every thread returns the same answer; false: the step was aborted.
__device__ __forceinline__ bool wg_poll16(const PArgs& a, Smem& S, const uint32_t* src, int n, bool pad3, uint32_t tag,
                                          bf16_t* dst, int ph) {
  const int tid = threadIdx.x;
  const int nw = pad3 ? p3_extent(n) : n;            // pad3: laid out by p3
  uint4 w[3];
  Waiter wt;
  while (true) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int q = tid + j * kPT;
      if (q * 4 < n) w[j] = get16x4(src, nw, pad3 ? p3(q * 4) : q * 4);
    }
    const uint32_t stw = tid == 0 ? get16(a.status) : 0u;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int q = tid + j * kPT;
      if (q * 4 < n)
        ok = ok && tag_ok(w[j].x, tag) && tag_ok(w[j].y, tag) && tag_ok(w[j].z, tag) && tag_ok(w[j].w, tag);
    }
    if (tid == 0) S.stop = wt.expired(stw) ? 1 : 0;
    if (__syncthreads_and(ok ? 1 : 0)) break;
    if (S.stop) {
      if (tid == 0) raise_abort(a, ph, wt.why, wt.polls);
      return false;
    }
  }
  DH_MARK(a, ph, 1);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int q = tid + j * kPT;
    if (q * 4 < n)
      *reinterpret_cast<uint2*>(dst + q * 4) = make_uint2((w[j].x >> 16) | (w[j].y & 0xffff0000u),
                                                          (w[j].z >> 16) | (w[j].w & 0xffff0000u));
  }
  return true;
}

// RMSNorm of the staged row in place, as the single-row GEMV kernel: sum of squares over the
// workgroup's threads (chunk stride kPT), DPP wave sums, the four wave sums in order.
__device__ __forceinline__ void norm_staged(Smem& S, int K, float eps) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nchunk = K / 8;
  float ss = 0.f;
  for (int i = tid; i < nchunk; i += kPT) {
    float xf[8];
    unpack8(S.sx[i], xf);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += xf[e] * xf[e];
  }
  ss = wave_sum(ss);
  if (lane == 0) S.red[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < kPW; ++w2) tot += S.red[w2];
  const float rs = rsqrtf(tot / (float)K + eps);
  for (int i = tid; i < nchunk; i += kPT) {
    float xf[8], gw[8];
    unpack8(S.sx[i], xf);
    unpack8(S.sg[i], gw);
#pragma unroll
    for (int e = 0; e < 8; ++e) xf[e] = rnd(xf[e] * rs * gw[e]);
    S.sx[i] = pack8(xf);
  }
  __syncthreads();
}

// The same wait for the x vector (n tagged words, n % 8 == 0, n <= 8 * kPT, laid out by xpos) with
// the eight words of thread i (chunks 2i and 2i + 1) polled by thread i (two 16-byte loads) and
// returned in its registers (xc, bf16); threads past the row only take part in the rounds' barriers.
__device__ __forceinline__ bool wg_poll16_chunk(const PArgs& a, Smem& S, const uint32_t* src, int n, uint32_t tag,
                                                uint4& xc, int ph) {
  const int tid = threadIdx.x;
  const bool mine = tid * 8 < n;
  const int nw = n / 4 * kXSeg;                      // padded extent
  uint4 w0 = make_uint4(0u, 0u, 0u, 0u), w1 = w0;
  Waiter wt;
  while (true) {
    bool ok = true;
    if (mine) {
      w0 = get16x4(src, nw, (2 * tid) * kXSeg);
      w1 = get16x4(src, nw, (2 * tid + 1) * kXSeg);
    }
    const uint32_t stw = tid == 0 ? get16(a.status) : 0u;
    if (mine)
      ok = tag_ok(w0.x, tag) && tag_ok(w0.y, tag) && tag_ok(w0.z, tag) && tag_ok(w0.w, tag) && tag_ok(w1.x, tag) &&
           tag_ok(w1.y, tag) && tag_ok(w1.z, tag) && tag_ok(w1.w, tag);
    if (tid == 0) S.stop = wt.expired(stw) ? 1 : 0;
    if (__syncthreads_and(ok ? 1 : 0)) break;
    if (S.stop) {
      if (tid == 0) raise_abort(a, ph, wt.why, wt.polls);
      return false;
    }
  }
  DH_MARK(a, ph, 1);
  xc = make_uint4((w0.x >> 16) | (w0.y & 0xffff0000u), (w0.z >> 16) | (w0.w & 0xffff0000u),
                  (w1.x >> 16) | (w1.y & 0xffff0000u), (w1.z >> 16) | (w1.w & 0xffff0000u));
  return true;
}

// norm_staged for a row whose chunk i thread i holds in registers (K <= 8 * kPT): the same sums
// (chunk i's squares in order, DPP wave sums, the kPW wave sums in order) and rounding; the
// normalised chunks go to the staged row. One barrier fewer, and no round trip of the raw row
// through LDS.
__device__ __forceinline__ void norm_chunk_regs(Smem& S, int K, float eps, const uint4& xc) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nchunk = K / 8;
  const bool mine = tid < nchunk;
  float xf[8];
  unpack8(xc, xf);
  float ss = 0.f;
  if (mine) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += xf[e] * xf[e];
  }
  ss = wave_sum(ss);
  if (lane == 0) S.red[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < kPW; ++w2) tot += S.red[w2];
  const float rs = rsqrtf(tot / (float)K + eps);
  if (mine) {
    float gw[8];
    unpack8(S.sg[tid], gw);
#pragma unroll
    for (int e = 0; e < 8; ++e) xf[e] = rnd(xf[e] * rs * gw[e]);
    S.sx[tid] = pack8(xf);
  }
  __syncthreads();
}

// A row of K <= 4 * kPT bf16 elements held four per thread (requested with a phase's weights) into
// the staged row or the norm-weight region of LDS.
__device__ __forceinline__ void stage_regs(uint4* dst, uint2 v, int K) {
  if ((int)threadIdx.x * 4 < K) reinterpret_cast<uint2*>(dst)[threadIdx.x] = v;
}
__device__ __forceinline__ uint2 fetch_row4(const bf16_t* src, int K) {
  return ld8(src + (int64_t)min((int)threadIdx.x * 4, K - 4));
}

// the dot products of R rows (CG chunks per lane) with the staged row
template <int R, int NW, int CG>
__device__ __forceinline__ void dot_rows(const Smem& S, int nchunk, const uint4 (&w)[R][NW][CG], float (&acc)[R][NW]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < NW; ++q) acc[r][q] = 0.f;
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const bool live = lane + 64 * c < nchunk;
    const uint4 hx = S.sx[min(lane + 64 * c, nchunk - 1)];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        const float sdot = dot8_bf16(w[r][q][c], hx);
        acc[r][q] += live ? sdot : 0.f;
      }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < NW; ++q) acc[r][q] = wave_sum(acc[r][q]);
}

template <int R, int NW, int CG>
__device__ __forceinline__ void load_rows(uint4 (&w)[R][NW][CG], const bf16_t* const (&rows)[R][NW], int nchunk) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int ch = min(lane + 64 * c, nchunk - 1);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q) w[r][q][c] = ldw16(rows[r][q] + (int64_t)ch * 8);
  }
}

// ---- the layer input: tagged x (or the embedding row, x0, for the first layer), normalised with
// the norm weight g (both requested with the phase's weights)
__device__ __forceinline__ bool stage_input(const PArgs& a, Smem& S, bool first, uint2 x0, uint2 g, uint32_t xtag, int ph) {
  stage_regs(S.sg, g, a.d);
  if (first) {
    stage_regs(S.sx, x0, a.d);
    DH_MARK(a, ph, 1);
    __syncthreads();
    norm_staged(S, a.d, a.eps);
  } else {
    uint4 xc;
    if (!wg_poll16_chunk(a, S, a.xw, a.d, xtag, xc, ph)) return false;
    norm_chunk_regs(S, a.d, a.eps, xc);
  }
  return true;
}

// The residual of output row n. The x phases (tree out-projection, attention out-projection, down
// projection) give row n to global wave n, so the wave that adds the residual of row n produced it
// in the previous x phase and keeps it in a register (xres); before the first x phase xres holds
// the embedding row's element n, loaded when the step starts.
__device__ __forceinline__ float residual(bool, const bf16_t*, int, float xres) { return xres; }

// ---------------------------------------------------------------------------------------------
// GEMV phases
// ---------------------------------------------------------------------------------------------
// The phases are split in two: fetch_* requests what a phase reads that no workgroup of this
// launch writes (weight rows, ring values, cached keys and values, history rows) into registers,
// run_* waits for the phase's inputs and computes. The kernel issues the fetch of phase p + 1
// before it runs phase p, so a phase's weights stream in during the previous phase's wait.

// Row groups of the GEMV phases: R rows per wave of NW matrices, CG 16-byte chunks per lane
template <int R, int NW, int CG>
struct Rows {
  uint4 w[R][NW][CG];
};
template <int R, int NW, int CG>
__device__ __forceinline__ void fetch_rows(Rows<R, NW, CG>& f, const bf16_t* const (&rows)[R][NW], int nchunk) {
  load_rows<R, NW, CG>(f.w, rows, nchunk);
}

// first phase of a layer (in-projection / q,k,v: 3 rows per wave, K = d) or the vocabulary head's
// first group (4 rows per wave): one register shape for both, so the fetch for "the next layer's
// first phase" has one type
struct PreFirst : Rows<4, 1, 2> {
  uint2 g;                         // the RMSNorm weight (norm1, or norm_out for the head), 4 per thread
  uint2 x0;                        // the first layer: the token's embedding row, 4 per thread
};

// RMSNorm + [W_a; W_b; W_c] rows of global wave gw: base row gw * 3 of N = n0 + n1 + n2
__device__ __forceinline__ void fetch_in3(PreFirst& f, const PArgs& a, int n0, int n1, int n2, const bf16_t* W0,
                                          const bf16_t* W1, const bf16_t* W2) {
  constexpr int R = 3;
  const int N = n0 + n1 + n2;
  const int base = (blockIdx.x * kPW + (threadIdx.x >> 6)) * R;
  const int nchunk = a.d / 8, lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < R; ++r) {                       // the fourth slot of the shared shape stays unused
    const int n = min(base + r, N - 1);
    const bf16_t* W = n < n0 ? W0 : (n < n0 + n1 ? W1 : W2);
    const int loc = n < n0 ? n : (n < n0 + n1 ? n - n0 : n - n0 - n1);
#pragma unroll
    for (int c = 0; c < 2; ++c) f.w[r][0][c] = ldw16(W + (int64_t)loc * a.d + (int64_t)min(lane + 64 * c, nchunk - 1) * 8);
  }
}

// Segments 0 and 1 go to the tagged in-projection group (global row n at p3(n)); segment 2 to
// `plain2` (the B_hist row of t) or the group. The launch has at least N / 3 waves.
__device__ __forceinline__ bool run_in3(const PArgs& a, Smem& S, const PreFirst& f, bool first,
                                        uint32_t xtag, int ph, Tags tg, bf16_t* plain2, int n0, int n1, int n2) {
  constexpr int R = 3, CG = 2;                        // K = d <= 1024
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = n0 + n1 + n2;
  const int nchunk = a.d / 8;
  const int base = (blockIdx.x * kPW + wave) * R;
  if (blockIdx.x * kPW * R >= N) return true;         // uniform: no rows in this workgroup
  if (!stage_input(a, S, first, f.x0, f.g, xtag, ph)) return false;
  if (base >= N) return true;                          // uniform per wave
  uint4 w[R][1][CG];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < CG; ++c) w[r][0][c] = f.w[r][0][c];
  float acc[R][1];
  dot_rows<R, 1, CG>(S, nchunk, w, acc);
  if (lane < R && base + lane < N) {
    float v0 = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) v0 = r == lane ? acc[r][0] : v0;
    const int n = base + lane;
    const float out = rnd(v0);
    if (n >= n0 + n1 && plain2) st2(plain2 + (n - n0 - n1), f32_to_bf16(out));
    else put16(a.i3w + p3(n), out, tg.t16(ph));
  }
  return true;
}

// RMSNorm2 + SwiGLU(W_gate, W_up) -> tagged h (ff words), R = 3 rows per wave
struct PreUp : Rows<3, 2, 2> {
  uint2 g;                         // norm2, 4 per thread
};
__device__ __forceinline__ void fetch_ffn_up(PreUp& f, const PArgs& a, LayerRef Lt) {
  constexpr int R = 3;
  const int N = a.ff;
  const int base = (blockIdx.x * kPW + (threadIdx.x >> 6)) * R;
  const bf16_t* Wg = (const bf16_t*)(intptr_t)Lt[F_WGATE];
  const bf16_t* Wu = (const bf16_t*)(intptr_t)Lt[F_WUP];
  f.g = fetch_row4((const bf16_t*)(intptr_t)Lt[F_NORM2], a.d);
  const bf16_t* rows[R][2];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(base + r, N - 1);
    rows[r][0] = Wg + (int64_t)n * a.d;
    rows[r][1] = Wu + (int64_t)n * a.d;
  }
  fetch_rows<3, 2, 2>(f, rows, a.d / 8);
}
__device__ __forceinline__ bool run_ffn_up(const PArgs& a, Smem& S, const PreUp& f, LayerRef Lt, uint32_t xtag,
                                           int ph, Tags tg) {
  constexpr int R = 3, CG = 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = a.ff, nchunk = a.d / 8;
  const int base = (blockIdx.x * kPW + wave) * R;
  if (blockIdx.x * kPW * R >= N) return true;
  stage_regs(S.sg, f.g, a.d);
  uint4 xc;
  if (!wg_poll16_chunk(a, S, a.xw, a.d, xtag, xc, ph)) return false;
  norm_chunk_regs(S, a.d, a.eps, xc);
  if (base >= N) return true;
  float acc[R][2];
  dot_rows<R, 2, CG>(S, nchunk, f.w, acc);
  if (lane < R && base + lane < N) {
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v0 = r == lane ? acc[r][0] : v0;
      v1 = r == lane ? acc[r][1] : v1;
    }
    put16(a.hw + p3(base + lane), rnd(rnd(silu(rnd(v0))) * rnd(v1)), tg.t16(ph));
  }
  return true;
}

// out[n] = round(round(W[n] . in) + resid[n]) -> tagged x, one row per wave (the launch has at
// least d waves); `in` is a tagged vector of K words (h for the down projection, y for attention's
// output projection)
template <int CG>
__device__ __forceinline__ void fetch_row(Rows<1, 1, CG>& f, const bf16_t* W, int K, int N) {
  const int n = blockIdx.x * kPW + (threadIdx.x >> 6);
  const bf16_t* rows[1][1] = {{W + (int64_t)min(n, N - 1) * K}};
  fetch_rows<1, 1, CG>(f, rows, K / 8);
}
template <int CG>
__device__ __forceinline__ bool run_rows_resid(const PArgs& a, Smem& S, const Rows<1, 1, CG>& f, int K,
                                               const uint32_t* in, bool in_pad3, uint32_t in_tag, bool first,
                                               const bf16_t* erow, float& xres, int ph, Tags tg) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = a.d, nchunk = K / 8;
  const int n = blockIdx.x * kPW + wave;
  if (blockIdx.x * kPW >= N) return true;
  if (!wg_poll16(a, S, in, K, in_pad3, in_tag, reinterpret_cast<bf16_t*>(S.sx), ph)) return false;
  __syncthreads();
  if (n >= N) return true;
  const float rv = residual(first, erow, n, xres);
  float acc[1][1];
  dot_rows<1, 1, CG>(S, nchunk, f.w, acc);
  xres = rnd(rnd(acc[0][0]) + rv);
  if (lane == 0) put16(a.xw + xpos(n), xres, tg.t16(ph));
  return true;
}

// ---------------------------------------------------------------------------------------------
// Tree layer: gate readouts (one wave per (level, head)), then the recurrence + out-projection
// ---------------------------------------------------------------------------------------------
struct PreGates {                 // raw words: converting them here would wait for the loads
  uint4 w[3][2];
  uint4 bv[2];
  uint32_t bi, bf, br, rsrc;
};
// the wave's (level, head) unit: u = global wave (H * L units over >= H * L waves)
__device__ __forceinline__ void fetch_gates(PreGates& f, const PArgs& a, LayerRef Lt, int64_t t) {
  constexpr int C = 2;                                // GH <= 1024
  const int lane = threadIdx.x & 63;
  const int u = blockIdx.x * kPW + (threadIdx.x >> 6);
  const int H = a.H, L = a.L, GH = a.GH;
  const int uu = min(u, H * L - 1);
  const int h = uu % H, l = uu / H;
  const int nchunk = GH / 8;
  const int64_t wrow = ((int64_t)l * H + h) * GH;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t k = (int64_t)min(lane + 64 * c, nchunk - 1) * 8;
    f.w[0][c] = ldw16((const bf16_t*)(intptr_t)Lt[F_WI] + wrow + k);
    f.w[1][c] = ldw16((const bf16_t*)(intptr_t)Lt[F_WF] + wrow + k);
    f.w[2][c] = ldw16((const bf16_t*)(intptr_t)Lt[F_WR] + wrow + k);
  }
  const int64_t gi = (int64_t)l * H + h;
  f.bi = ld2((const bf16_t*)(intptr_t)Lt[F_BI] + gi);
  f.bf = ld2((const bf16_t*)(intptr_t)Lt[F_BF] + gi);
  f.br = ld2((const bf16_t*)(intptr_t)Lt[F_BR] + gi);
  const int64_t src = t - ((int64_t)1 << l);
  const int64_t sc = src >= 0 ? src : 0;
#pragma unroll
  for (int c = 0; c < C; ++c)
    f.bv[c] = ld16((const bf16_t*)(intptr_t)Lt[F_BHIST] + sc * GH + (int64_t)min(lane + 64 * c, nchunk - 1) * 8);
  f.rsrc = ld2((const bf16_t*)(intptr_t)Lt[F_RGHIST] + (sc * L + l) * H + h);
}

__device__ __forceinline__ void run_gates(const PArgs& a, Smem& S, const PreGates& f, LayerRef Lt, int64_t t,
                                          uint32_t atag, int ph, Tags tg) {
  constexpr int C = 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int u = blockIdx.x * kPW + (tid >> 6);
  const int H = a.H, L = a.L, GH = a.GH;
  if (blockIdx.x * kPW >= H * L) return;               // uniform: no unit in this workgroup
  const int nchunk = GH / 8;                           // <= kPT
  // A polled once per workgroup (thread i: chunk i, 8 tagged words) into LDS, instead of by every
  // wave: a quarter of the poll traffic, and the workgroup's waves see A in the same round
  {
    const bool mine = tid < nchunk;
    const uint32_t tg16 = tg.t16(atag);
    uint4 p0 = make_uint4(0u, 0u, 0u, 0u), p1 = p0;
    Waiter wt;
    while (true) {
      bool okw = true;
      if (mine) {
        p0 = get16x4(a.i3w, a.n3w, p3(a.d + tid * 8));
        p1 = get16x4(a.i3w, a.n3w, p3(a.d + tid * 8 + 4));
      }
      const uint32_t stw = tid == 0 ? get16(a.status) : 0u;   // with the data: no extra round trip
      if (mine)
        okw = tag_ok(p0.x, tg16) && tag_ok(p0.y, tg16) && tag_ok(p0.z, tg16) && tag_ok(p0.w, tg16) &&
              tag_ok(p1.x, tg16) && tag_ok(p1.y, tg16) && tag_ok(p1.z, tg16) && tag_ok(p1.w, tg16);
      if (tid == 0) S.stop = wt.expired(stw) ? 1 : 0;
      if (__syncthreads_and(okw ? 1 : 0)) break;
      if (S.stop) {
        if (tid == 0) raise_abort(a, ph, wt.why, wt.polls);
        return;
      }
    }
    DH_MARK(a, ph, 1);
    if (mine)
      S.sx[tid] = make_uint4((p0.x >> 16) | (p0.y & 0xffff0000u), (p0.z >> 16) | (p0.w & 0xffff0000u),
                             (p1.x >> 16) | (p1.y & 0xffff0000u), (p1.z >> 16) | (p1.w & 0xffff0000u));
    __syncthreads();
  }
  if (u >= H * L) return;                              // uniform per wave
  const int h = u % H, l = u / H;
  const int64_t src = t - ((int64_t)1 << l);
  const bool ok = src >= 0;
  uint4 av[C];
#pragma unroll
  for (int c = 0; c < C; ++c) av[c] = S.sx[min(lane + 64 * c, nchunk - 1)];
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float wi[8], wf[8], wr[8], x1[8], x2[8];
    unpack8(f.w[0][c], wi);
    unpack8(f.w[1][c], wf);
    unpack8(f.w[2][c], wr);
    unpack8(av[c], x1);
    unpack8(f.bv[c], x2);
    const float live = (lane + 64 * c) < nchunk ? 1.f : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
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
  if (lane == 0) {
    const float okf = ok ? 1.f : 0.f;
    const float ig = dh_sigmoid(s0 + bfv(f.bi)) * okf;
    const float fg = dh_sigmoid(s1 + bfv(f.bf)) * okf + (1.f - okf);
    const float rs = ok ? bfv(f.rsrc) : 0.f;
    // records in unit order (u = l * H + h): a workgroup's four units fill one 64-byte segment
    put32(a.coefw + (int64_t)u * 2, fg, tg.t32(ph));
    put32(a.coefw + (int64_t)u * 2 + 1, ig * rs, tg.t32(ph));
    st2((bf16_t*)(intptr_t)Lt[F_RGHIST] + (t * L + l) * H + h, f32_to_bf16(dh_sigmoid(s2 + bfv(f.br))));
  }
}

// Every workgroup runs the L-level recurrence of all d elements (4 per thread) from the ring
// sources (requested before the wait) and the tagged gates and V0; workgroup 0 writes the ring
// slots of t and Y. Then one out-projection row per wave plus the residual -> tagged x.
struct PreScan {
  Rows<1, 1, 2> w;                 // this wave's out-projection row
  uint2 vs[kLMax];                 // raw ring sources of this thread's four elements, per level
};
__device__ __forceinline__ void fetch_scan(PreScan& f, const PArgs& a, LayerRef Lt, int64_t t) {
  const int d = a.d, L = a.L;
  const int e0 = min((int)threadIdx.x * 4, d - 4);
  const bf16_t* ring = (const bf16_t*)(intptr_t)Lt[F_VRING];
  fetch_row<2>(f.w, (const bf16_t*)(intptr_t)Lt[F_WOUT], d, d);
#pragma unroll
  for (int l = 0; l < kLMax; ++l) {
    const int lc = min(l, L - 1);
    const int64_t src = t - ((int64_t)1 << lc);
    const int64_t scl = src >= 0 ? src : 0;
    f.vs[l] = ld8(ring + (ring_offset(lc) + (scl & ring_mask(lc))) * d + e0);
  }
}

__device__ __forceinline__ bool run_scan_out(const PArgs& a, Smem& S, const PreScan& f, LayerRef Lt, int64_t t,
                                             bool first, const bf16_t* erow, float& xres, int v0ph, int gph, int ph,
                                             Tags tg, void* Yout) {
  constexpr int CG = 2;                               // d <= 1024
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int H = a.H, L = a.L, hd = a.hd, d = a.d;
  const int nchunk = d / 8;
  const int e0 = min(tid * 4, d - 4);
  const int h = e0 / hd;
  const bf16_t* ring = (const bf16_t*)(intptr_t)Lt[F_VRING];
  const int n = blockIdx.x * kPW + wave;             // one row per wave (d rows over >= d waves)
  float vs[kLMax][4];
#pragma unroll
  for (int l = 0; l < kLMax; ++l) {
    const int lc = min(l, L - 1);
    const bool ok = t - ((int64_t)1 << lc) >= 0;
    const float q4[4] = {bfv(f.vs[l].x & 0xffffu), bfv(f.vs[l].x >> 16), bfv(f.vs[l].y & 0xffffu), bfv(f.vs[l].y >> 16)};
#pragma unroll
    for (int q = 0; q < 4; ++q) vs[l][q] = ok ? q4[q] : 0.f;
  }
  // ---- one wait for the gates (a 16-byte pair per (head, level), into LDS) and this thread's four
  // V0 words (straight into registers)
  float v[4], v0f[4];
  {
    const int ncf = H * L;                             // <= 3 * kPT
    const uint32_t* cw32 = reinterpret_cast<const uint32_t*>(a.coefw);
    const uint32_t gt = tg.t32(gph), vt = tg.t16(v0ph);
    uint4 cw[3], vw;
    Waiter wt;
    while (true) {
      const uint32_t stw = tid == 0 ? get16(a.status) : 0u;
      bool ok = true;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int i = tid + j * kPT;
        if (i < ncf) {
          cw[j] = get16x4(cw32, ncf * 4, i * 4);
          ok = ok && cw[j].y == gt && cw[j].w == gt;
        }
      }
      vw = get16x4(a.i3w, a.n3w, p3(e0));
      ok = ok && tag_ok(vw.x, vt) && tag_ok(vw.y, vt) && tag_ok(vw.z, vt) && tag_ok(vw.w, vt);
      if (tid == 0) S.stop = wt.expired(stw) ? 1 : 0;
      if (__syncthreads_and(ok ? 1 : 0)) break;
      if (S.stop) {
        if (tid == 0) raise_abort(a, ph, wt.why, wt.polls);
        return false;
      }
    }
    DH_MARK(a, ph, 1);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int i = tid + j * kPT;                     // record i: unit (level i / H, head i % H)
      if (i < ncf) S.coef[(i % H) * L + i / H] = make_float2(__uint_as_float(cw[j].x), __uint_as_float(cw[j].z));
    }
    v0f[0] = bfv(vw.x >> 16); v0f[1] = bfv(vw.y >> 16); v0f[2] = bfv(vw.z >> 16); v0f[3] = bfv(vw.w >> 16);
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = v0f[q];
  float hist[kLMax][4];
#pragma unroll
  for (int l = 0; l < kLMax; ++l) {
    const bool on = l < L;
    const float2 cf = S.coef[h * L + min(l, L - 1)];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float nv = __builtin_fmaf(cf.y, vs[l][q], cf.x * v[q]);   // as dh_decode_scan_out
      v[q] = on ? nv : v[q];
      hist[l][q] = v[q];
    }
  }
  if (tid * 4 < d) {
    *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(S.sx) + e0) =
        make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                   (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
  }
  __syncthreads();
  if (n < d) {
    const float rv = residual(first, erow, n, xres);
    float acc[1][1];
    dot_rows<1, 1, CG>(S, nchunk, f.w.w, acc);
    xres = rnd(rnd(acc[0][0]) + rv);
    if (lane == 0) put16(a.xw + xpos(n), xres, tg.t16(ph));
  }
  // the ring slots of t are read by later launches only: workgroup 0 writes them after its x rows
  // are out, so they do not queue ahead of the hand-off
  if (blockIdx.x == 0 && tid * 4 < d) {
    bf16_t* rw = (bf16_t*)ring + e0;
    auto st4 = [](bf16_t* p, const float (&x)[4]) {
      st8(p, make_uint2((uint32_t)f32_to_bf16(x[0]) | ((uint32_t)f32_to_bf16(x[1]) << 16),
                        (uint32_t)f32_to_bf16(x[2]) | ((uint32_t)f32_to_bf16(x[3]) << 16)));
    };
    st4(rw + (t & 1) * d, v0f);
#pragma unroll
    for (int l = 0; l + 1 < kLMax; ++l)
      if (l + 1 < L) st4(rw + (ring_offset(l + 1) + (t & ring_mask(l + 1))) * d, hist[l]);
    if (Yout) st4((bf16_t*)Yout + e0, v);
  }
  return true;
}

// ---------------------------------------------------------------------------------------------
// Attention layer: split-window segments (16 per head, two per workgroup of 128 threads each),
// then one workgroup per head combines the segment records.
// ---------------------------------------------------------------------------------------------
// geometry of this thread's attention segment unit (two units of kUT threads per workgroup)
struct AttnGeo {
  int un, ut, lane, wave, sg, h, lo, nw, P, j0, j1, jc1;
  bool live, has_t;
  bf16_t *Kh, *Vh;
};
__device__ __forceinline__ AttnGeo attn_geo(const PArgs& a, LayerRef Lt, int64_t t) {
  AttnGeo g;
  const int tid = threadIdx.x;
  g.un = tid / kUT;
  g.ut = tid % kUT;
  g.lane = tid & 63;
  g.wave = g.ut >> 6;
  const int u = blockIdx.x * 2 + g.un;
  g.live = u < a.H * kSplitS;
  const int uu = g.live ? u : 0;
  g.sg = uu % kSplitS;
  g.h = uu / kSplitS;
  const int window = (int)Lt[F_WINDOW];
  g.lo = window > 0 ? (int)max((int64_t)0, t + 1 - window) : 0;
  g.nw = (int)t - g.lo + 1;
  g.P = (g.nw + kSplitS - 1) / kSplitS;
  g.j0 = min(g.sg * g.P, g.nw);
  g.j1 = min(g.nw, g.j0 + g.P);
  g.has_t = g.live && g.j0 <= g.nw - 1 && g.nw - 1 < g.j1;
  g.jc1 = g.live ? min(g.j1, g.nw - 1) : g.j0;
  const int64_t head_off = (int64_t)g.h * a.Tmax * kHD;
  g.Kh = (bf16_t*)(intptr_t)Lt[F_KC] + head_off;
  g.Vh = (bf16_t*)(intptr_t)Lt[F_VC] + head_off;
  return g;
}

struct PreAttn {
  uint4 krow[kHD / 8];             // the unit's first key rows (one per thread)
  uint4 vrow[8];                   // its first value rows (lane -> (row slot, chunk))
  uint32_t rc, rsn;                // raw rotation operands of t
};
__device__ __forceinline__ void fetch_attn(PreAttn& f, const PArgs& a, LayerRef Lt, int64_t t) {
  constexpr int VE = 8, KCH = kHD / VE, RPI = 64 / KCH, NW = kUT / 64, VCH = 8;
  const AttnGeo g = attn_geo(a, Lt, t);
  const int pt = min(g.ut, kHD / 2 - 1);
  f.rc = ld2((const bf16_t*)(intptr_t)Lt[F_COS] + t * (kHD / 2) + pt);
  f.rsn = ld2((const bf16_t*)(intptr_t)Lt[F_SIN] + t * (kHD / 2) + pt);
  const int i = g.j0 + g.ut;
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    f.krow[c] = make_uint4(0u, 0u, 0u, 0u);
    if (i < g.jc1 && g.P <= kMaxSeg) f.krow[c] = ld16(g.Kh + (int64_t)(g.lo + i) * kHD + c * 8);
  }
  const int slot = g.lane / KCH, dg = g.lane % KCH;
#pragma unroll
  for (int q = 0; q < VCH; ++q) {
    const int iv = g.j0 + (q * NW + g.wave) * RPI + slot;
    f.vrow[q] = make_uint4(0u, 0u, 0u, 0u);
    if (iv < g.jc1 && g.P <= kMaxSeg) f.vrow[q] = ld16(g.Vh + (int64_t)(g.lo + iv) * kHD + dg * 8);
  }
}

__device__ __forceinline__ bool run_attn_split(const PArgs& a, Smem& S, const PreAttn& f, LayerRef Lt, int64_t t,
                                               int qph, int ph, Tags tg) {
  constexpr int VE = 8, KCH = kHD / VE, RPI = 64 / KCH, NW = kUT / 64, VCH = 8;
  const int tid = threadIdx.x;
  if (blockIdx.x * 2 >= a.H * kSplitS) return true;   // uniform
  const AttnGeo g = attn_geo(a, Lt, t);
  const int un = g.un, ut = g.ut, lane = g.lane, wave = g.wave, sg = g.sg, h = g.h, lo = g.lo, nw_ = g.nw;
  const int j0 = g.j0, j1 = g.j1, jc1 = g.jc1;
  const bool unit_live = g.live, has_t = g.has_t;
  bf16_t* Kh = g.Kh;
  bf16_t* Vh = g.Vh;
  if (g.P > kMaxSeg) {                                 // uniform: the window's segment exceeds the LDS scores
    if (tid == 0) raise_abort(a, ph);
    return false;
  }
  const float scale = sqrtf((float)kHD);
  const int pt = min(ut, kHD / 2 - 1);
  const uint32_t rc = f.rc, rsn = f.rsn;
  uint4 krow[KCH], vrow[VCH];
#pragma unroll
  for (int c = 0; c < KCH; ++c) krow[c] = f.krow[c];
#pragma unroll
  for (int q = 0; q < VCH; ++q) vrow[q] = f.vrow[q];
  const int slot = lane / KCH, dg = lane % KCH;
  // ---- q, k, v of this head (tagged): threads < 32 of a unit hold one rotation pair
  bool dead = false;
  const bool roper = ut < kHD / 2;
  const int base = h * kHD + 2 * pt;
  const uint32_t tq = tg.t16(qph);
  float q0 = 0.f, q1 = 0.f, k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
  {
    Waiter wt;
    uint32_t wq0 = 0, wq1 = 0, wk0 = 0, wk1 = 0, wv0 = 0, wv1 = 0;
    while (true) {
      const uint32_t stw = tid == 0 ? get16(a.status) : 0u;
      bool ok = true;
      if (roper && unit_live) {
        const int pq = p3(base), pk = p3(a.d + base), pv = p3(2 * a.d + base);   // base even: +1 stays in its chunk
        wq0 = get16(a.i3w + pq); wq1 = get16(a.i3w + pq + 1);
        wk0 = get16(a.i3w + pk); wk1 = get16(a.i3w + pk + 1);
        wv0 = get16(a.i3w + pv); wv1 = get16(a.i3w + pv + 1);
        ok = tag_ok(wq0, tq) && tag_ok(wq1, tq) && tag_ok(wk0, tq) && tag_ok(wk1, tq) && tag_ok(wv0, tq) && tag_ok(wv1, tq);
      }
      if (tid == 0) S.stop = wt.expired(stw) ? 1 : 0;
      if (__syncthreads_and(ok ? 1 : 0)) break;
      if (S.stop) {
        if (tid == 0) raise_abort(a, ph, wt.why, wt.polls);
        return false;
      }
    }
    DH_MARK(a, ph, 1);
    q0 = bfv(wq0 >> 16); q1 = bfv(wq1 >> 16);
    k0 = bfv(wk0 >> 16); k1 = bfv(wk1 >> 16);
    v0 = bfv(wv0 >> 16); v1 = bfv(wv1 >> 16);
  }
  if (roper && unit_live) {
    const float c = bfv(rc), s = bfv(rsn);
    float qr0, qr1, kr0, kr1;
    {
#pragma clang fp contract(off)
      qr0 = rnd(rnd(q0 * c) - rnd(q1 * s));
      qr1 = rnd(rnd(q0 * s) + rnd(q1 * c));
      kr0 = rnd(rnd(k0 * c) - rnd(k1 * s));
      kr1 = rnd(rnd(k0 * s) + rnd(k1 * c));
    }
    S.qs[un][2 * ut] = qr0; S.qs[un][2 * ut + 1] = qr1;
    S.ks[un][2 * ut] = kr0; S.ks[un][2 * ut + 1] = kr1;
    S.vsh[un][2 * ut] = v0; S.vsh[un][2 * ut + 1] = v1;
    if (has_t) {
      st2(Kh + t * kHD + 2 * ut, f32_to_bf16(kr0));
      st2(Kh + t * kHD + 2 * ut + 1, f32_to_bf16(kr1));
      st2(Vh + t * kHD + 2 * ut, f32_to_bf16(v0));
      st2(Vh + t * kHD + 2 * ut + 1, f32_to_bf16(v1));
    }
  }
  __syncthreads();

  // ---- scores of the cached positions and of t
  const float* qs = S.qs[un];
  auto score = [&](const uint4 (&w)[KCH]) {
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const uint32_t wsd[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
      const int e = c * VE;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dot += qs[e + 2 * j] * __uint_as_float(wsd[j] << 16) + qs[e + 2 * j + 1] * __uint_as_float(wsd[j] & 0xffff0000u);
    }
    return rnd(rnd(dot) / scale);
  };
  float* sc = S.sc[un];
  float mx = -INFINITY;
  for (int i0 = j0; i0 < jc1; i0 += kUT) {
    const int i = i0 + ut;
    if (i0 > j0 && i < jc1) {
#pragma unroll
      for (int c = 0; c < KCH; ++c) krow[c] = ld16(Kh + (int64_t)(lo + i) * kHD + c * 8);
    }
    const float s0 = score(krow);
    if (i < jc1) {
      sc[i - j0] = s0;
      mx = fmaxf(mx, s0);
    }
  }
  if (has_t && ut == 0) {
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < kHD; ++e) dot += qs[e] * S.ks[un][e];
    const float s2 = rnd(rnd(dot) / scale);
    sc[nw_ - 1 - j0] = s2;
    mx = fmaxf(mx, s2);
  }
  mx = wave_max(mx);
  if (lane == 0) S.ared[un][wave] = mx;
  __syncthreads();
  float M = S.ared[un][0];
#pragma unroll
  for (int w2 = 1; w2 < NW; ++w2) M = fmaxf(M, S.ared[un][w2]);
  __syncthreads();
  float sum = 0.f;
  for (int i = j0 + ut; i < j1 && unit_live; i += kUT) {
    const float p = __expf(sc[i - j0] - M);
    sc[i - j0] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  if (lane == 0) S.ared[un][wave] = sum;
  __syncthreads();
  float Ls = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) Ls += S.ared[un][w2];

  // ---- o = sum p_i V_i
  float acc[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) acc[e] = 0.f;
  auto accumulate = [&](const uint4& w, int i) {
    if (i >= jc1) return;
    const float p = sc[i - j0];
    const uint32_t wsd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] += p * __uint_as_float(wsd[j] << 16);
      acc[2 * j + 1] += p * __uint_as_float(wsd[j] & 0xffff0000u);
    }
  };
#pragma unroll
  for (int q = 0; q < VCH; ++q) accumulate(vrow[q], j0 + (q * NW + wave) * RPI + slot);
  for (int i0 = j0 + VCH * NW * RPI; i0 < jc1; i0 += VCH * NW * RPI) {
#pragma unroll
    for (int q = 0; q < VCH; ++q) {
      const int i = i0 + (q * NW + wave) * RPI + slot;
      if (i < jc1) vrow[q] = ld16(Vh + (int64_t)(lo + i) * kHD + dg * 8);
    }
#pragma unroll
    for (int q = 0; q < VCH; ++q) accumulate(vrow[q], i0 + (q * NW + wave) * RPI + slot);
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
    for (int e = 0; e < VE; ++e) S.part[un][wave][dg * VE + e] = acc[e];
  }
  __syncthreads();
  if (unit_live) {
    uint64_t* rec = a.partw + ((int64_t)h * kSplitS + sg) * kRecW;
    if (ut < kHD) {
      float o = has_t ? sc[nw_ - 1 - j0] * S.vsh[un][ut] : 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) o += S.part[un][w2][ut];
      put32(rec + 2 + ut, o, tg.t32(ph));
    }
    if (ut == 0) {
      put32(rec, M, tg.t32(ph));
      put32(rec + 1, Ls, tg.t32(ph));
    }
  }
  return true;
}

// one workgroup per head: y[h*64 + e] = round(sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s) -> tagged y.
// The four waves poll four segments each (eight loads a lane per round instead of 32 for one
// wave), the records meet in LDS, and wave 0 forms y with the same sums, in the same order, as
// the combine launch of the graph of launches.
static_assert(kSplitS == 4 * kPW, "four segments per wave");
__device__ __forceinline__ void phase_attn_combine(const PArgs& a, Smem& S, int sph, int ph, Tags tg) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if ((int)blockIdx.x >= a.H) return;                  // uniform
  const int h = blockIdx.x, e = lane;
  const uint64_t* rec = a.partw + (int64_t)h * kSplitS * kRecW;
  const uint32_t* rec32 = reinterpret_cast<const uint32_t*>(rec);
  const int nw32 = kSplitS * kRecW * 2;
  const uint32_t st = tg.t32(sph);
  float m4[4], l4[4], o4[4];
  {
    Waiter wt;
    while (true) {
      const uint32_t stw = tid == 0 ? get16(a.status) : 0u;
      bool ok = true;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int sg = 4 * wave + q;
        const uint4 ml = get16x4(rec32, nw32, sg * kRecW * 2);         // m, l of segment sg
        const uint64_t ow = get32(rec + sg * kRecW + 2 + e);
        ok = ok && ml.y == st && ml.w == st && (uint32_t)(ow >> 32) == st;
        m4[q] = __uint_as_float(ml.x);
        l4[q] = __uint_as_float(ml.z);
        o4[q] = __uint_as_float((uint32_t)ow);
      }
      if (tid == 0) S.stop = wt.expired(stw) ? 1 : 0;
      if (__syncthreads_and(ok ? 1 : 0)) break;
      if (S.stop) {
        if (tid == 0) raise_abort(a, ph, wt.why, wt.polls);
        return;
      }
    }
  }
  DH_MARK(a, ph, 1);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    S.co[4 * wave + q][e] = o4[q];
    if (e == 0) {
      S.cm[4 * wave + q] = m4[q];
      S.cl[4 * wave + q] = l4[q];
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float m[kSplitS];
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kSplitS; ++s) {
    m[s] = S.cm[s];
    M = fmaxf(M, m[s]);
  }
  float Lsum = 0.f, y = 0.f;
#pragma unroll
  for (int s = 0; s < kSplitS; ++s) {
    const float w = m[s] > -INFINITY ? __expf(m[s] - M) : 0.f;
    Lsum += w * S.cl[s];
    y += w * S.co[s][e];
  }
  put16(a.yw + h * kHD + e, y / Lsum, tg.t16(ph));
}

// ---------------------------------------------------------------------------------------------
// Vocabulary head and greedy pick
// ---------------------------------------------------------------------------------------------
// the vocabulary head's rows of group `base` (4 rows of global wave gw, groups 4 * waves apart).
// Ordinary loads, not the non-temporal ones of the layer weights: part of the head's 103 MB then
// survives in the memory-side cache until the next step's head (337.1 -> 335.2 us per token, one box)
__device__ __forceinline__ void fetch_head_rows(uint4 (&w)[4][1][2], const PArgs& a, int base) {
  const bf16_t* rows[4][1];
#pragma unroll
  for (int r = 0; r < 4; ++r) rows[r][0] = a.emb + (int64_t)min(base + r, a.V - 1) * a.d;
  const int lane = threadIdx.x & 63, nchunk = a.d / 8;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int ch = min(lane + 64 * c, nchunk - 1);
#pragma unroll
    for (int r = 0; r < 4; ++r) w[r][0][c] = ld16(rows[r][0] + (int64_t)ch * 8);
  }
}
__device__ __forceinline__ void fetch_lm_head(PreFirst& f, const PArgs& a) {
  fetch_head_rows(f.w, a, (blockIdx.x * kPW + (threadIdx.x >> 6)) * 4);
  f.g = fetch_row4(a.norm_out, a.d);
}

__device__ __forceinline__ bool run_lm_head(const PArgs& a, Smem& S, const PreFirst& f, uint32_t xtag, int ph, Tags tg) {
  constexpr int R = 4, CG = 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = a.V, K = a.d, nchunk = K / 8;
  const int gw = blockIdx.x * kPW + wave, nw = gridDim.x * kPW;
  float cv = -INFINITY;
  int ci = 0x7fffffff;
  // two row groups in flight: wa holds rows base (requested a phase ahead for the first group), wb
  // the next group of the stride, each refilled two groups ahead as soon as its dot products are done
  uint4 wa[R][1][CG], wb[R][1][CG];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < CG; ++c) wa[r][0][c] = f.w[r][0][c];
  const int stride = nw * R;
  stage_regs(S.sg, f.g, K);
  uint4 xc;
  if (!wg_poll16_chunk(a, S, a.xw, K, xtag, xc, ph)) return false;
  // requested after the poll: loads complete in issue order, so an earlier request would hold up
  // the poll's rounds
  if (gw * R + stride < N) fetch_head_rows(wb, a, gw * R + stride);
  norm_chunk_regs(S, K, a.eps, xc);
  auto group = [&](uint4 (&w)[R][1][CG], int base) {
    float acc[R][1];
    dot_rows<R, 1, CG>(S, nchunk, w, acc);
    if (base + 2 * stride < N) fetch_head_rows(w, a, base + 2 * stride);
    if (lane < R && base + lane < N) {
      float v0 = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) v0 = r == lane ? acc[r][0] : v0;
      const float out = rnd(v0);
      a.logits[base + lane] = f32_to_bf16(out);
      if (beats(out, base + lane, cv, ci)) {
        cv = out;
        ci = base + lane;
      }
    }
  };
  for (int base = gw * R; base < N; base += 2 * stride) {
    group(wa, base);
    if (base + stride < N) group(wb, base + stride);
  }
  wave_best(cv, ci);
  if (lane == 63) S.wbest[wave] = Cand{cv, ci};
  __syncthreads();
  if (threadIdx.x == 0) {
    Cand r = S.wbest[0];
#pragma unroll
    for (int w2 = 1; w2 < kPW; ++w2)
      if (beats(S.wbest[w2].v, S.wbest[w2].i, r.v, r.i)) r = S.wbest[w2];
    put32(a.candw + 8 * blockIdx.x, r.v, tg.t32(ph));      // a 64-byte segment per workgroup
    put32(a.candw + 8 * blockIdx.x + 1, __int_as_float(r.i), tg.t32(ph));
  }
  return true;
}

__device__ __forceinline__ void phase_argmax(const PArgs& a, Smem& S, int64_t t, int nph_lm, int ph, Tags tg) {
  if (blockIdx.x != 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  bool dead = false;
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  for (int i0 = 0; i0 < (int)gridDim.x; i0 += kPT) {
    const int i = i0 + tid;
    const bool want = i < (int)gridDim.x;
    float v = 0.f;
    int ix = 0;
    {
      const uint32_t* c32 = reinterpret_cast<const uint32_t*>(a.candw);
      const uint32_t ct = tg.t32(nph_lm);
      Waiter wt;
      while (!dead) {
        const uint32_t stw = get16(a.status);
        const uint4 cw = get16x4(c32, (int)gridDim.x * 16, min(i, (int)gridDim.x - 1) * 16);
        v = __uint_as_float(cw.x);
        ix = (int)cw.z;
        if (__all(!want || (cw.y == ct && cw.w == ct))) break;
        if (wt.expired(__builtin_amdgcn_readfirstlane(stw))) {
          raise_abort(a, ph, wt.why, wt.polls);
          dead = true;
        }
      }
    }
    if (want && beats(v, ix, best, bidx)) {
      best = v;
      bidx = ix;
    }
  }
  DH_MARK(a, ph, 1);
  wave_best(best, bidx);
  if (lane == 63) S.wbest[wave] = Cand{best, bidx};
  __syncthreads();
  if (tid == 0 && !dead && !aborted(a)) {
    Cand r = S.wbest[0];
#pragma unroll
    for (int w2 = 1; w2 < kPW; ++w2)
      if (beats(S.wbest[w2].v, S.wbest[w2].i, r.v, r.i)) r = S.wbest[w2];
    *a.token = r.i;
    if (a.tok_hist && t + 1 < a.hist_len) a.tok_hist[t + 1] = r.i;
    *a.t_dev = t + 1;
  }
  // The epoch advances at the end of every launch whose pick phase runs, also one that saw an
  // abort here; a workgroup 0 that left an earlier phase on an abort does not advance it, and the
  // host advances it when it clears the status (the status is sticky until then, so every launch
  // in between stops at its first wait).
  if (tid == 0) *a.epoch = *a.epoch + 1;
}

// the first phase of layer Lt: the tree in-projection [W_in; W_gh; W_ghs] or attention's [W_q; W_k; W_v]
__device__ __forceinline__ void fetch_first(PreFirst& f, const PArgs& a, LayerRef Lt, const bf16_t* erow) {
  f.g = fetch_row4((const bf16_t*)(intptr_t)Lt[F_NORM1], a.d);
  if (erow) f.x0 = fetch_row4(erow, a.d);
  if (Lt[F_KIND] == 0)
    fetch_in3(f, a, a.d, a.GH, a.GH, (const bf16_t*)(intptr_t)Lt[F_WIN], (const bf16_t*)(intptr_t)Lt[F_WGH],
              (const bf16_t*)(intptr_t)Lt[F_WGS]);
  else
    fetch_in3(f, a, a.d, a.d, a.d, (const bf16_t*)(intptr_t)Lt[F_WQ], (const bf16_t*)(intptr_t)Lt[F_WK],
              (const bf16_t*)(intptr_t)Lt[F_WV]);
}

// Phase order of a step (one per hand-off), each phase's fetch issued before the previous phase
// runs: tree layer I (in-projection) G (gate readouts) S (recurrence + out-projection), attention
// layer Q (q, k, v) A (window segments) C (combine) O (out-projection), then U, D (feed-forward
// up, down) in both, and after the last layer N (vocabulary head) M (greedy pick).
__global__ __launch_bounds__(kPT) void decode_persistent_kernel(PArgs a) {
  __shared__ Smem S;
  const int64_t t = load_uniform(a.t_dev);
  const int64_t tok = load_uniform(a.token);
  const int64_t ep = load_uniform(a.epoch);
  if (t < 0 || t >= a.Tmax) return;                   // uniform: nothing to do (the graphed step writes nothing either)
  const Tags tg{(uint64_t)ep * (uint64_t)a.nph};
  const bf16_t* erow = a.emb + (int64_t)tok * a.d;
  // the layer table, copied once into LDS (fields are then read without touching the vector-memory
  // counter the weight requests occupy)
  __shared__ int64_t s_tab[kMaxLayers * kLW];
  for (int i = threadIdx.x; i < a.n_layers * kLW; i += kPT) s_tab[i] = a.table[i];
  const int xrow = min((int)(blockIdx.x * kPW + (threadIdx.x >> 6)), a.d - 1);
  float xres = bf16_to_f32(ld2(erow + xrow));          // x[n] this wave last wrote (its x-phase row n)
  __syncthreads();
  const LayerRef tab0{(lds_i64*)s_tab};
  int ph = 0;
  int xph = -1;                                        // phase that last wrote x (-1: the embedding row)
  PreFirst pf;                                         // the next layer's first phase (then the head's)
  fetch_first(pf, a, tab0, erow);
  for (int li = 0; li < a.n_layers; ++li) {
    const LayerRef Lt{tab0.p + (int64_t)li * kLW};
    const bool first = xph < 0;
    const uint32_t xtag = first ? 0u : tg.t16(xph);
    PreUp pu;
    if (Lt[F_KIND] == 0) {
      PreGates pg;
      fetch_gates(pg, a, Lt, t);
      const int p_in = ph++;                           // V0, A (tagged), B_hist[t] (plain)
      DH_MARK(a, p_in, 0);
      if (!run_in3(a, S, pf, first, xtag, p_in, tg, (bf16_t*)(intptr_t)Lt[F_BHIST] + t * a.GH, a.d, a.GH, a.GH))
        return;
      DH_MARK(a, p_in, 2);
      PreScan ps;
      fetch_scan(ps, a, Lt, t);
      const int p_g = ph++;
      DH_MARK(a, p_g, 0);
      run_gates(a, S, pg, Lt, t, p_in, p_g, tg);
      DH_MARK(a, p_g, 2);
      fetch_ffn_up(pu, a, Lt);
      const int p_s = ph++;
      DH_MARK(a, p_s, 0);
      if (!run_scan_out(a, S, ps, Lt, t, first, erow, xres, p_in, p_g, p_s, tg, nullptr)) return;
      DH_MARK(a, p_s, 2);
      xph = p_s;
    } else {
      PreAttn pa;
      fetch_attn(pa, a, Lt, t);
      const int p_q = ph++;
      DH_MARK(a, p_q, 0);
      if (!run_in3(a, S, pf, first, xtag, p_q, tg, nullptr, a.d, a.d, a.d))
        return;
      DH_MARK(a, p_q, 2);
      const int p_a = ph++;
      DH_MARK(a, p_a, 0);
      if (!run_attn_split(a, S, pa, Lt, t, p_q, p_a, tg)) return;
      DH_MARK(a, p_a, 2);
      Rows<1, 1, 2> po;
      fetch_row<2>(po, (const bf16_t*)(intptr_t)Lt[F_WO], a.d, a.d);
      const int p_c = ph++;
      DH_MARK(a, p_c, 0);
      phase_attn_combine(a, S, p_a, p_c, tg);
      DH_MARK(a, p_c, 2);
      fetch_ffn_up(pu, a, Lt);
      const int p_o = ph++;
      DH_MARK(a, p_o, 0);
      if (!run_rows_resid<2>(a, S, po, a.d, a.yw, false, tg.t16(p_c), first, erow, xres, p_o, tg)) return;
      DH_MARK(a, p_o, 2);
      xph = p_o;
    }
    Rows<1, 1, 6> pd;
    fetch_row<6>(pd, (const bf16_t*)(intptr_t)Lt[F_WDOWN], a.ff, a.d);
    const int p_u = ph++;
    DH_MARK(a, p_u, 0);
    if (!run_ffn_up(a, S, pu, Lt, tg.t16(xph), p_u, tg)) return;
    DH_MARK(a, p_u, 2);
    if (li + 1 < a.n_layers) fetch_first(pf, a, Lt.next(), nullptr);
    else fetch_lm_head(pf, a);
    const int p_d = ph++;
    DH_MARK(a, p_d, 0);
    if (!run_rows_resid<6>(a, S, pd, a.ff, a.hw, true, tg.t16(p_u), false, erow, xres, p_d, tg)) return;
    DH_MARK(a, p_d, 2);
    xph = p_d;
  }
  const int p_n = ph++;
  DH_MARK(a, p_n, 0);
  if (!run_lm_head(a, S, pf, tg.t16(xph), p_n, tg)) return;
  DH_MARK(a, p_n, 2);
  const int p_m = ph++;
  DH_MARK(a, p_m, 0);
  phase_argmax(a, S, t, p_n, p_m, tg);
  DH_MARK(a, p_m, 2);
}

// phases of a step: 5 per tree layer, 6 per attention layer, 2 for the head and the pick
int count_phases(const int* kinds, int n) {
  int p = 2;
  for (int i = 0; i < n; ++i) p += kinds[i] == 0 ? 5 : 6;
  return p;
}

}  // namespace

extern "C" int64_t dh_decode_persistent_scratch_bytes(int d, int GH, int H, int L, int ff, int grid) {
  // tagged bf16 vectors: x, V0, A, h, q, k, v, y; fp32 records: gates, segment records, candidates
  // x (xpos), the in-projection group (p3 over max(d + GH, 3d) rows), h (p3), y
  const int64_t w16 = (int64_t)d / 4 * kXSeg + p3_extent(d + GH > 3 * d ? d + GH : 3 * d) + p3_extent(ff) + d;
  const int64_t w32 = ((int64_t)H * L * 2 + 7) / 8 * 8 + (int64_t)H * kSplitS * kRecW + (int64_t)8 * grid;
  return 256 + (w16 * 4 + 255) / 256 * 256 + w32 * 8 + 256;
}

namespace {
int launch_persistent(const char* who, const int64_t* layer_table, const int* kinds, int n_layers, const void* emb,
                      const void* norm_out, float eps, int d, int GH, int H, int hd, int L, int ff, int V, int Tmax,
                      int64_t* t_dev, int64_t* token, int64_t* tok_hist, int64_t hist_len, void* logits,
                      void* scratch, int64_t scratch_bytes, uint64_t* trace, int64_t trace_words, void* stream) {
  DH_REQUIRE(layer_table && kinds && emb && norm_out && t_dev && token && logits && scratch, DH_ERR_INVALID_ARG,
             "%s: null pointer argument", who);
  DH_REQUIRE(n_layers >= 1 && n_layers <= kMaxLayers, DH_ERR_UNSUPPORTED_SHAPE, "%s: %d layers (1..%d)", who,
             n_layers, kMaxLayers);
  DH_REQUIRE(d >= 256 && d <= 1024 && d % 256 == 0 && H * hd == d && GH >= 64 && GH <= 1024 && GH % 64 == 0 &&
                 ff >= 64 && ff <= 3072 && ff % 32 == 0 && L >= 1 && L <= kLMax && H * L <= 64 * kLMax,
             DH_ERR_UNSUPPORTED_SHAPE, "%s: d=%d H=%d hd=%d GH=%d ff=%d L=%d not supported", who, d, H, hd, GH, ff, L);
  DH_REQUIRE(V >= 1 && Tmax >= 1 && hist_len >= 0, DH_ERR_INVALID_ARG, "%s: V=%d Tmax=%d", who, V, Tmax);
  int dev = 0, ncu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return dh_fail(DH_ERR_LAUNCH_FAILED, "%s: cannot query the device", who);
  const int grid = ncu;
  DH_REQUIRE(grid * kPW >= d && grid * kPW * 3 >= d + 2 * GH && grid * kPW * 3 >= ff && grid * 2 >= H * kSplitS && grid * kPW >= H * L &&
                 grid <= kPT,
             DH_ERR_UNSUPPORTED_SHAPE, "%s: %d compute units do not fit d=%d GH=%d ff=%d", who, grid, d, GH, ff);
  bool has_attn = false;
  for (int i = 0; i < n_layers; ++i) {
    DH_REQUIRE(kinds[i] == 0 || kinds[i] == 1, DH_ERR_INVALID_ARG, "%s: layer %d kind %d", who, i, kinds[i]);
    has_attn |= kinds[i] == 1;
  }
  DH_REQUIRE(!has_attn || hd == kHD, DH_ERR_UNSUPPORTED_SHAPE, "%s: attention head width %d (needs %d)", who, hd, kHD);
  const int64_t need = dh_decode_persistent_scratch_bytes(d, GH, H, L, ff, grid);
  DH_REQUIRE(scratch_bytes >= need && ((uintptr_t)scratch % 256) == 0, DH_ERR_INVALID_ARG,
             "%s: scratch of %lld bytes (256-byte aligned) needed, %lld given", who, (long long)need,
             (long long)scratch_bytes);
  PArgs a{};
  a.table = layer_table;
  a.n_layers = n_layers;
  a.emb = (const bf16_t*)emb;
  a.norm_out = (const bf16_t*)norm_out;
  a.t_dev = t_dev;
  a.token = token;
  a.tok_hist = tok_hist;
  a.hist_len = hist_len;
  a.logits = (bf16_t*)logits;
  a.eps = eps;
  a.d = d; a.GH = GH; a.H = H; a.hd = hd; a.L = L; a.ff = ff; a.V = V; a.Tmax = Tmax;
  a.nph = count_phases(kinds, n_layers);
  DH_REQUIRE(!trace || trace_words >= (int64_t)grid * a.nph * 3, DH_ERR_INVALID_ARG,
             "%s: trace of %lld words, needs %lld (CUs x phases x 3)", who, (long long)trace_words,
             (long long)grid * a.nph * 3);
  a.trace = trace;
  char* p = (char*)scratch;
  a.epoch = (int64_t*)p;
  a.status = (uint32_t*)(p + 8);
  uint32_t* w = (uint32_t*)(p + 256);
  a.n3w = p3_extent(d + GH > 3 * d ? d + GH : 3 * d);
  a.nhw = p3_extent(ff);
  a.xw = w; w += d / 4 * kXSeg;
  a.i3w = w; w += a.n3w;
  a.hw = w; w += a.nhw;
  a.yw = w; w += d;
  uint64_t* r = (uint64_t*)(p + 256 + ((int64_t)(w - (uint32_t*)(p + 256)) * 4 + 255) / 256 * 256);
  a.coefw = r; r += ((int64_t)H * L * 2 + 7) / 8 * 8;   // regions start on 64-byte boundaries
  a.partw = r; r += (int64_t)H * kSplitS * kRecW;
  a.candw = r;
  // One workgroup per compute unit, all resident: the kernel's registers (>256 VGPRs over four
  // waves) admit at most one workgroup per CU, so a launch of exactly one per CU on an idle device
  // (stream order: the previous step has drained) places every workgroup at once. A plain launch
  // (not hipLaunchCooperativeKernel, which added ~20 us between steps) also records into graphs.
  // Should a workgroup ever not be resident, the bounded waits end the step with the status set.
  static int occ_checked = -1;
  if (occ_checked < 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&decode_persistent_kernel),
                                                     kPT, 0) != hipSuccess)
      return dh_fail(DH_ERR_LAUNCH_FAILED, "%s: occupancy query failed", who);
    occ_checked = per_cu;
  }
  DH_REQUIRE(occ_checked >= 1, DH_ERR_LAUNCH_FAILED, "%s: the kernel does not fit a compute unit", who);
  decode_persistent_kernel<<<dim3(grid), dim3(kPT), 0, (hipStream_t)stream>>>(a);
  return dh_check_launch(who);
}
}  // namespace

extern "C" int dh_decode_persistent_step(const int64_t* layer_table, const int* kinds, int n_layers, const void* emb,
                                         const void* norm_out, float eps, int d, int GH, int H, int hd, int L, int ff,
                                         int V, int Tmax, int64_t* t_dev, int64_t* token, int64_t* tok_hist,
                                         int64_t hist_len, void* logits, void* scratch, int64_t scratch_bytes,
                                         void* stream) {
  return launch_persistent("dh_decode_persistent_step", layer_table, kinds, n_layers, emb, norm_out, eps, d, GH, H, hd,
                           L, ff, V, Tmax, t_dev, token, tok_hist, hist_len, logits, scratch, scratch_bytes, nullptr, 0,
                           stream);
}

extern "C" int dh_decode_persistent_trace(const int64_t* layer_table, const int* kinds, int n_layers, const void* emb,
                                          const void* norm_out, float eps, int d, int GH, int H, int hd, int L, int ff,
                                          int V, int Tmax, int64_t* t_dev, int64_t* token, int64_t* tok_hist,
                                          int64_t hist_len, void* logits, void* scratch, int64_t scratch_bytes,
                                          uint64_t* trace, int64_t trace_words, void* stream) {
  DH_REQUIRE(trace, DH_ERR_INVALID_ARG, "dh_decode_persistent_trace: null trace");
  return launch_persistent("dh_decode_persistent_trace", layer_table, kinds, n_layers, emb, norm_out, eps, d, GH, H,
                           hd, L, ff, V, Tmax, t_dev, token, tok_hist, hist_len, logits, scratch, scratch_bytes, trace,
                           trace_words, stream);
}

extern "C" int dh_decode_persistent_phases(const int* kinds, int n_layers) { return count_phases(kinds, n_layers); }

extern "C" int dh_decode_persistent_status(const void* scratch, uint32_t* out2, void* stream) {
  DH_REQUIRE(scratch && out2, DH_ERR_INVALID_ARG, "dh_decode_persistent_status: null pointer argument");
  const hipError_t e = hipMemcpyAsync(out2, (const char*)scratch + 8, 8, hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e != hipSuccess) return dh_fail(DH_ERR_LAUNCH_FAILED, "dh_decode_persistent_status: %s", hipGetErrorString(e));
  if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
    return dh_fail(DH_ERR_LAUNCH_FAILED, "dh_decode_persistent_status: stream synchronisation failed");
  return 0;
}
