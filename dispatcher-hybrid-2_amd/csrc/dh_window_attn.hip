// Banded (sliding-window) causal attention for the parallel forward and the decoder prefill, gfx950.
//
// Semantics (reference dispatcher_hybrid/modeling_dispatcher.py:163-166 rope, :168-182 forward):
//   q', k'  = rope(q[t]), rope(k[t])      interleaved pairs (x0 c - x1 s, x0 s + x1 c) at position t
//   y[t]    = sum_s softmax_s(q'[t] . k'[s] / sqrt(hd)) v[s]   over  s <= t  and  t - s < window
//             (window 0: every s <= t)
// with the eager bf16 path's rounding where it defines stored state: each rope product and sum
// rounded (so the cache rows below are the eager prefill's bit for bit); scores stay fp32 (the
// eager path rounds them to bf16 first: the kernel is the more accurate of the two), softmax in
// fp32, probabilities rounded to bf16 for the value product, output rounded once. The softmax is
// evaluated online over key blocks (running max and sum, the output rescaled per block), so it
// normalises at the end where the eager path normalises first: outputs agree to bf16 rounding,
// not bit for bit.
// Two launches: a pre-pass writes rope(k) and v of every position to (B, H, Tmax, hd) buffers --
// the decoder caches (reference dispatcher_hybrid/decoding.py:143-185, attention part) or scratch --
// so each key is rotated once; the attention kernel reads its key and value blocks from there
// (each block of 64 keys is 64 contiguous rows of one head).
//
// Work decomposition: a workgroup of 4 waves owns 64 queries of one (batch row, head); wave w owns
// queries q0 + 16w .. +15. The key blocks of the band (64 keys each) are staged in LDS -- keys
// row-major with rows padded to hd*2 + 16 bytes; values transposed (hd rows of 64 keys, padded to
// 136 bytes) -- double-buffered, the next block's global loads in flight during the current
// block. Scores are computed transposed, S^T = K Q^T (v_mfma_f32_16x16x32_bf16, A = key
// rows from LDS, B = the wave's rotated query fragments held in registers), so the C fragment puts
// one query per lane column: the running max, sum and rescale stay per lane (plus two cross-group
// shuffles per reduction), and the probabilities are already in the B-operand layout of
// O^T = V^T P^T, whose A operand reads the transposed values from LDS. Workgroups are numbered so
// consecutive query blocks of one (batch row, head) run on one XCD (round-robin dispatch: block id
// mod 8), sharing the band's key and value lines in that XCD's L2.
#include "dh_common.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kBQ = 64;          // queries per workgroup
constexpr int kBK = 64;          // keys per block
constexpr int kThreads = 256;

struct WinArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  int64_t sb, st;               // batch and position strides of q, k, v (elements)
  const bf16_t* cos;            // (>= T, hd/2)
  const bf16_t* sin;
  bf16_t* y;
  int64_t yb, yt;
  bf16_t* kc;                   // nullable caches (B, H, Tmax, hd)
  bf16_t* vc;
  int64_t cb, ch;               // cache batch / head strides (elements); rows hd apart
  int B, T, H, window, nq, nwork;
  float scale2;                 // 1/sqrt(hd) * log2(e): scores go to the log2 domain
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const void* p) { return *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// bf16 rounding through the compiler's conversion (v_cvt_pk_bf16_f32: round to nearest even, the
// rounding torch's bf16 ops use); a pair packs in one instruction
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float rnd(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  bf16x2_t v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// rope of 8 consecutive elements (4 interleaved pairs) with their 4 cos / sin values; every product
// and sum rounded to bf16 on its own (torch evaluates them as separate bf16 tensor ops)
__device__ __forceinline__ uint4 rope8(const uint4& x, const uint2& c, const uint2& s) {
  const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
  const float cv[4] = {lo_f(c.x), hi_f(c.x), lo_f(c.y), hi_f(c.y)};
  const float sv[4] = {lo_f(s.x), hi_f(s.x), lo_f(s.y), hi_f(s.y)};
  uint32_t o[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float e = lo_f(xw[p]), d = hi_f(xw[p]);
    float r0, r1;
    {
#pragma clang fp contract(off)
      r0 = rnd(rnd(e * cv[p]) - rnd(d * sv[p]));
      r1 = rnd(rnd(e * sv[p]) + rnd(d * cv[p]));
    }
    o[p] = pack2(r0, r1);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// Pre-pass: rope(k) and v of every position into the (B, H, Tmax, hd) buffers the attention reads
// (the decoder caches, or scratch): each key is rotated once, not by every workgroup whose band
// holds it. One thread per 16-byte chunk.
template <int HD>
__global__ __launch_bounds__(kThreads) void rope_kv_kernel(WinArgs a) {
  constexpr int CPR = HD / 8;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t n = (int64_t)a.B * a.T * a.H * CPR;
  if (i >= n) return;
  const int c = (int)(i % CPR);
  const int64_t row = i / CPR;                   // (b, t, h) in that order: reads are contiguous
  const int h = (int)(row % a.H);
  const int64_t bt = row / a.H;
  const int t = (int)(bt % a.T), b = (int)(bt / a.T);
  const int64_t src = (int64_t)b * a.sb + (int64_t)t * a.st + (int64_t)h * HD + 8 * c;
  const uint4 kr = rope8(ld16(a.k + src), ld8(a.cos + (int64_t)t * (HD / 2) + 4 * c),
                         ld8(a.sin + (int64_t)t * (HD / 2) + 4 * c));
  const int64_t dst = (int64_t)b * a.cb + (int64_t)h * a.ch + (int64_t)t * HD + 8 * c;
  *reinterpret_cast<uint4*>(a.kc + dst) = kr;
  *reinterpret_cast<uint4*>(a.vc + dst) = ld16(a.v + src);
}

template <int HD>
__global__ __launch_bounds__(kThreads) void window_attn_kernel(WinArgs a) {
  constexpr int KROW = HD * 2 + 16;              // padded key row (bytes)
  constexpr int VROW = kBK * 2 + 8;              // padded transposed-value row (bytes)
  constexpr int KS = HD / 32;                    // MFMA k-steps over hd
  constexpr int NT = HD / 16;                    // hd tiles of the output
  constexpr int CPR = HD / 8;                    // 16-byte chunks per row
  constexpr int LPT = kBK * CPR / kThreads;      // key (and value) chunks per thread per block
  static_assert(LPT >= 1 && kBK * CPR % kThreads == 0, "block shape");
  // with two or more chunks a thread takes pairs of consecutive keys at one column, so the
  // transposed values are written as 4-byte (key, key + 1) words
  constexpr bool PAIRS = LPT % 2 == 0;
  __shared__ __align__(16) unsigned char ks[2][kBK * KROW];
  __shared__ __align__(16) unsigned char vt[2][HD * VROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  // work item: consecutive items (query blocks of one (b, h)) on one XCD
  const int per = (a.nwork + 7) >> 3;
  const int w = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (w >= a.nwork) return;
  const int qb = w % a.nq, bh = w / a.nq;
  const int h = bh % a.H, b = bh / a.H;
  const int q0 = qb * kBQ;
  const int tq = q0 + wave * 16 + r;             // this lane's query
  const bf16_t* qp = a.q + (int64_t)b * a.sb + (int64_t)h * HD;
  const bf16_t* kp = a.kc + (int64_t)b * a.cb + (int64_t)h * a.ch;    // rotated keys, rows of hd
  const bf16_t* vp = a.vc + (int64_t)b * a.cb + (int64_t)h * a.ch;

  // ---- K/V block staging. Chunk i of the thread -> (key, 16-byte column): without pairs chunk
  // index tid + 256 i -> key idx / CPR, column idx % CPR; with pairs, pair tid + 256 (i / 2) ->
  // keys 2 (idx / CPR) + (i & 1), column idx % CPR
  auto chunk_of = [&](int i, int& key, int& c) {
    if constexpr (PAIRS) {
      const int idx = tid + (i >> 1) * kThreads;
      key = 2 * (idx / CPR) + (i & 1);
      c = idx % CPR;
    } else {
      const int idx = tid + i * kThreads;
      key = idx / CPR;
      c = idx % CPR;
    }
  };
  uint4 kraw[LPT], vraw[LPT];
  auto kv_fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      int key, c;
      chunk_of(i, key, c);
      const int t = min(kb * kBK + key, a.T - 1);
      kraw[i] = ld16(kp + (int64_t)t * HD + 8 * c);
      vraw[i] = ld16(vp + (int64_t)t * HD + 8 * c);
    }
  };
  auto kv_store = [&](int buf, int kb) {
    (void)kb;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      int key, c;
      chunk_of(i, key, c);
      *reinterpret_cast<uint4*>(&ks[buf][key * KROW + c * 16]) = kraw[i];
      const uint32_t vw[4] = {vraw[i].x, vraw[i].y, vraw[i].z, vraw[i].w};
      if constexpr (PAIRS) {
        if (i & 1) {                               // chunk i - 1 holds key - 1 at the same column
          const uint32_t uw[4] = {vraw[i - 1].x, vraw[i - 1].y, vraw[i - 1].z, vraw[i - 1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t lo = (e & 1) ? (uw[e >> 1] >> 16) : (uw[e >> 1] & 0xffffu);
            const uint32_t hi = (e & 1) ? (vw[e >> 1] & 0xffff0000u) : (vw[e >> 1] << 16);
            *reinterpret_cast<uint32_t*>(&vt[buf][(8 * c + e) * VROW + (key - 1) * 2]) = lo | hi;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<bf16_t*>(&vt[buf][(8 * c + e) * VROW + key * 2]) =
              (bf16_t)((e & 1) ? (vw[e >> 1] >> 16) : (vw[e >> 1] & 0xffffu));
      }
    }
  };

  // ---- rotated query fragments: lane (query r, k-group g) holds q'[tq][32 s + 8 g .. + 8]
  bf16x8 qf[KS];
  {
    const int tc = min(tq, a.T - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int col = 32 * s + 8 * g;
      const uint4 x = ld16(qp + (int64_t)tc * a.st + col);
      qf[s] = as_bf16x8(rope8(x, ld8(a.cos + (int64_t)tc * (HD / 2) + col / 2),
                              ld8(a.sin + (int64_t)tc * (HD / 2) + col / 2)));
    }
  }

  const int kb_lo = a.window > 0 ? max(0, q0 - a.window + 1) / kBK : 0;
  const int kb_hi = min(q0 + kBQ - 1, a.T - 1) / kBK;
  f32x4 o[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, l = 0.f;                      // running max (finite floor) and sum of this query

  kv_fetch(kb_lo);
  kv_store(0, kb_lo);
  __syncthreads();
  for (int kb = kb_lo; kb <= kb_hi; ++kb) {
    const int buf = (kb - kb_lo) & 1;
    const bool more = kb < kb_hi;                 // uniform
    if (more) kv_fetch(kb + 1);

    // ---- S^T = K Q^T: C fragment = query r (column), keys 16 tau + 4 g + i (rows)
    f32x4 sT[4];
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
      sT[tau] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&ks[buf][(tau * 16 + r) * KROW + (32 * s + 8 * g) * 2]);
        sT[tau] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[s], sT[tau], 0, 0, 0);
      }
    }
    // scores in the log2 domain (scale * log2 e folded in; softmax via 2^x). A block strictly below
    // the diagonal and wholly inside every query's window needs no mask (all blocks but the band's
    // first and last): a uniform branch.
    const bool interior = kb < qb && (a.window == 0 || q0 + kBQ - 1 - kb * kBK < a.window);
    float p[16];
    float mx = -INFINITY;
    if (interior) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        p[j] = sT[j >> 2][j & 3] * a.scale2;
        mx = fmaxf(mx, p[j]);
      }
    } else {
#pragma unroll
      for (int tau = 0; tau < 4; ++tau)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb * kBK + tau * 16 + 4 * g + i;
          const bool ok = key <= tq && key < a.T && (a.window == 0 || tq - key < a.window);
          const float sc = sT[tau][i] * a.scale2;
          p[tau * 4 + i] = ok ? sc : -INFINITY;
          mx = fmaxf(mx, p[tau * 4 + i]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      p[j] = __builtin_amdgcn_exp2f(p[j] - mn);   // masked: 2^-inf = 0
      ps += p[j];
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l = l * alpha + ps;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[nt][i] *= alpha;

    // ---- O^T += V^T P^T over the two 32-key steps; key order within a step: the lane group's
    // four keys of tile 2kk, then its four keys of tile 2kk + 1 (the same order on both operands)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint4 pw = make_uint4(pack2(p[(2 * kk) * 4 + 0], p[(2 * kk) * 4 + 1]),
                                  pack2(p[(2 * kk) * 4 + 2], p[(2 * kk) * 4 + 3]),
                                  pack2(p[(2 * kk + 1) * 4 + 0], p[(2 * kk + 1) * 4 + 1]),
                                  pack2(p[(2 * kk + 1) * 4 + 2], p[(2 * kk + 1) * 4 + 3]));
      const bf16x8 pf = as_bf16x8(pw);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const unsigned char* vrow = &vt[buf][(nt * 16 + r) * VROW];
        const uint2 v0 = *reinterpret_cast<const uint2*>(vrow + (32 * kk + 4 * g) * 2);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + (32 * kk + 16 + 4 * g) * 2);
        o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(make_uint4(v0.x, v0.y, v1.x, v1.y)), pf,
                                                        o[nt], 0, 0, 0);
      }
    }
    if (more) kv_store(buf ^ 1, kb + 1);
    __syncthreads();
  }

  // ---- output: lane holds query tq, hd columns 16 nt + 4 g + i
  if (tq < a.T) {
    const float inv = 1.f / l;
    bf16_t* yp = a.y + (int64_t)b * a.yb + (int64_t)tq * a.yt + (int64_t)h * HD;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      *reinterpret_cast<uint2*>(yp + nt * 16 + 4 * g) =
          make_uint2(pack2(o[nt][0] * inv, o[nt][1] * inv), pack2(o[nt][2] * inv, o[nt][3] * inv));
  }
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

}  // namespace

extern "C" int dh_window_attention_fwd(int dtype, const void* q, const void* k, const void* v, int64_t stride_b,
                                       int64_t stride_t, const void* rope_cos, const void* rope_sin, void* y,
                                       int64_t y_stride_b, int64_t y_stride_t, void* K_cache, void* V_cache,
                                       int64_t cache_stride_b, int64_t cache_stride_h, int Tmax, int B, int T, int H,
                                       int hd, int window, void* stream) {
  const char* who = "dh_window_attention_fwd";
  DH_REQUIRE(dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d (bf16 only)", who, dtype);
  DH_REQUIRE(hd == 32 || hd == 64 || hd == 128, DH_ERR_UNSUPPORTED_SHAPE, "%s: hd=%d not in {32,64,128}", who, hd);
  DH_REQUIRE(B >= 1 && T >= 1 && H >= 1 && window >= 0, DH_ERR_INVALID_ARG, "%s: B=%d T=%d H=%d window=%d", who, B,
             T, H, window);
  DH_REQUIRE(q && k && v && rope_cos && rope_sin && y, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(K_cache && V_cache, DH_ERR_INVALID_ARG, "%s: K_cache and V_cache are required", who);
  DH_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(y, 8) && stride_b % 8 == 0 &&
                 stride_t % 8 == 0 && y_stride_b % 4 == 0 && y_stride_t % 4 == 0 && stride_t >= (int64_t)H * hd &&
                 y_stride_t >= (int64_t)H * hd && aligned(rope_cos, 8) && aligned(rope_sin, 8),
             DH_ERR_INVALID_ARG, "%s: q/k/v rows need 16-byte and y rows 8-byte alignment", who);
  DH_REQUIRE(T <= Tmax && aligned(K_cache, 16) && aligned(V_cache, 16) && cache_stride_b % 8 == 0 &&
                 cache_stride_h % 8 == 0 && cache_stride_h >= (int64_t)Tmax * hd,
             DH_ERR_INVALID_ARG, "%s: caches (B, H, Tmax, hd) need T <= Tmax and 16-byte rows", who);
  const int nq = (T + kBQ - 1) / kBQ;
  const int64_t nwork = (int64_t)nq * H * B;
  DH_REQUIRE(nwork < (1 << 30), DH_ERR_UNSUPPORTED_SHAPE, "%s: too many query blocks", who);
  WinArgs a{(const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, stride_b, stride_t,
            (const bf16_t*)rope_cos, (const bf16_t*)rope_sin, (bf16_t*)y, y_stride_b, y_stride_t,
            (bf16_t*)K_cache, (bf16_t*)V_cache, cache_stride_b, cache_stride_h, B, T, H, window, nq, (int)nwork,
            (float)(1.0 / sqrt((double)hd)) * 1.44269504088896341f};   // torch's fp32 1/sqrt(hd), times log2 e
  const int grid = (int)(((nwork + 7) / 8) * 8);
  const int64_t chunks = (int64_t)B * T * H * (hd / 8);
  const int pgrid = (int)((chunks + kThreads - 1) / kThreads);
  hipStream_t s = (hipStream_t)stream;
  if (hd == 32) {
    rope_kv_kernel<32><<<dim3(pgrid), dim3(kThreads), 0, s>>>(a);
    window_attn_kernel<32><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  } else if (hd == 64) {
    rope_kv_kernel<64><<<dim3(pgrid), dim3(kThreads), 0, s>>>(a);
    window_attn_kernel<64><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  } else {
    rope_kv_kernel<128><<<dim3(pgrid), dim3(kThreads), 0, s>>>(a);
    window_attn_kernel<128><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  }
  return dh_check_launch(who);
}
