// Parallel gate pre-activations (and their backward) for gfx950.
//
// Forward semantics (reference dispatcher_hybrid/fused_gates.py:38-93 and the eager definition at
// dispatcher_hybrid/modeling_dispatcher.py:100-109):
//   ok[b,t,l]      = t < T && t >= 2^l && (mask == null || mask[b,t,l] > 0)
//   hid[b,t,l,k]   = relu(A[b,t,k] + ok * B[b,t-2^l,k])^2
//   pre_x[b,t,l,h] = sum_k hid[b,t,l,k] * W_x[l,h,k] + b_x[l,h]          x in {i, f, r}
// bf16 mode rounds a+b and hid to bf16 (the points where the eager bf16 path rounds), multiplies
// on bf16 MFMA with fp32 accumulation, adds the fp32 bias and rounds once on store. fp32 mode uses
// fp32 MFMA throughout.
//
// Work decomposition: one workgroup (4 wave64s) per (batch row, 64-position tile); wave w owns
// positions 16w..16w+15 of the tile and walks every level, so the A tile is fetched from HBM once
// and re-read per level from L2. For each level the hidden tile is formed directly in the MFMA
// A-operand registers (lane -> row lane%16, k-chunk lane/16) from A[t] and the lagged B[t-2^l] row,
// and multiplied against W_x[l] (the B operand: lane -> head lane%16, same k-chunk) for the three
// gates: N = 16 heads per MFMA tile, ceil(H/16) tiles per gate.
#include "dh_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTileT = 64;

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

struct FwdArgs {
  const void* A;
  const void* B;
  int64_t sab, sat;
  const void* Wi;
  const void* Wf;
  const void* Wr;
  int64_t swl, swh;
  const float* bi;
  const float* bf;
  const float* br;
  const void* mask;
  int64_t smb, smt;
  void* oi;
  void* of;
  void* orr;
  int b, T, GH, H, n_lv;
};

template <typename T>
__device__ __forceinline__ bool mask_ok(const FwdArgs& a, int b, int t, int l) {
  if (!a.mask) return true;
  return Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)t * a.smt + l) > 0.f;
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// bf16 forward
__global__ __launch_bounds__(kThreads) void gate_preacts_fwd_bf16(FwdArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int b = blockIdx.y;
  const int t = blockIdx.x * kTileT + wave * 16 + r;  // row this lane feeds into the MFMA
  const bool t_ok = t < a.T;
  const bf16_t* Ab = (const bf16_t*)a.A + (int64_t)b * a.sab;
  const bf16_t* Bb = (const bf16_t*)a.B + (int64_t)b * a.sab;
  const int NT = (a.H + 15) >> 4;

  for (int l = 0; l < a.n_lv; ++l) {
    const int src = t - (1 << l);
    const bool ok = t_ok && src >= 0 && mask_ok<bf16_t>(a, b, t, l);
    const bf16_t* Arow = Ab + (int64_t)(t_ok ? t : 0) * a.sat;
    const bf16_t* Brow = Bb + (int64_t)(ok ? src : 0) * a.sat;
    const int64_t wl = (int64_t)l * a.swl;
    for (int nt = 0; nt < NT; ++nt) {
      const int n = nt * 16 + r;  // head whose weights this lane feeds
      const bool n_ok = n < a.H;
      const int64_t wrow = wl + (int64_t)(n_ok ? n : 0) * a.swh;
      const bf16_t* wi = (const bf16_t*)a.Wi + wrow;
      const bf16_t* wf = (const bf16_t*)a.Wf + wrow;
      const bf16_t* wr = (const bf16_t*)a.Wr + wrow;
      f32x4 ci = {0.f, 0.f, 0.f, 0.f}, cf = ci, cr = ci;

      for (int k0 = 0; k0 < a.GH; k0 += 32) {
        const int kk = k0 + g * 8;
        uint4 av = t_ok ? ld16(Arow + kk) : make_uint4(0, 0, 0, 0);
        uint4 bv = ok ? ld16(Brow + kk) : make_uint4(0, 0, 0, 0);
        uint4 vi = n_ok ? ld16(wi + kk) : make_uint4(0, 0, 0, 0);
        uint4 vf = n_ok ? ld16(wf + kk) : make_uint4(0, 0, 0, 0);
        uint4 vr = n_ok ? ld16(wr + kk) : make_uint4(0, 0, 0, 0);
        const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
        const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
        bf16x8 hid;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a0 = __uint_as_float(aw[j] << 16), a1 = __uint_as_float(aw[j] & 0xffff0000u);
          const float b0 = __uint_as_float(bw[j] << 16), b1 = __uint_as_float(bw[j] & 0xffff0000u);
          float x0 = fmaxf(bf16_to_f32(f32_to_bf16(a0 + b0)), 0.f);
          float x1 = fmaxf(bf16_to_f32(f32_to_bf16(a1 + b1)), 0.f);
          hid[2 * j] = (short)f32_to_bf16(x0 * x0);
          hid[2 * j + 1] = (short)f32_to_bf16(x1 * x1);
        }
        bf16x8 wiv, wfv, wrv;
        __builtin_memcpy(&wiv, &vi, 16);
        __builtin_memcpy(&wfv, &vf, 16);
        __builtin_memcpy(&wrv, &vr, 16);
        ci = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hid, wiv, ci, 0, 0, 0);
        cf = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hid, wfv, cf, 0, 0, 0);
        cr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hid, wrv, cr, 0, 0, 0);
      }
      // C fragment: column (head) lane%16, rows 4*(lane/16) + i
      if (n_ok) {
        const float bvi = a.bi[l * a.H + n], bvf = a.bf[l * a.H + n], bvr = a.br[l * a.H + n];
        const int tb = blockIdx.x * kTileT + wave * 16 + g * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int to = tb + i;
          if (to < a.T) {
            const int64_t o = (((int64_t)b * a.T + to) * a.n_lv + l) * a.H + n;
            ((bf16_t*)a.oi)[o] = f32_to_bf16(ci[i] + bvi);
            ((bf16_t*)a.of)[o] = f32_to_bf16(cf[i] + bvf);
            ((bf16_t*)a.orr)[o] = f32_to_bf16(cr[i] + bvr);
          }
        }
      }
    }
  }
}

// fp32 forward: 16x16x4 fp32 MFMA; each lane loads 4 consecutive k and issues 4 MFMAs, lane group
// g covering k = k0 + 4g + j for MFMA j, on both operands.
__global__ __launch_bounds__(kThreads) void gate_preacts_fwd_f32(FwdArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int b = blockIdx.y;
  const int t = blockIdx.x * kTileT + wave * 16 + r;
  const bool t_ok = t < a.T;
  const float* Ab = (const float*)a.A + (int64_t)b * a.sab;
  const float* Bb = (const float*)a.B + (int64_t)b * a.sab;
  const int NT = (a.H + 15) >> 4;

  for (int l = 0; l < a.n_lv; ++l) {
    const int src = t - (1 << l);
    const bool ok = t_ok && src >= 0 && mask_ok<float>(a, b, t, l);
    const float* Arow = Ab + (int64_t)(t_ok ? t : 0) * a.sat;
    const float* Brow = Bb + (int64_t)(ok ? src : 0) * a.sat;
    const int64_t wl = (int64_t)l * a.swl;
    for (int nt = 0; nt < NT; ++nt) {
      const int n = nt * 16 + r;
      const bool n_ok = n < a.H;
      const int64_t wrow = wl + (int64_t)(n_ok ? n : 0) * a.swh;
      const float* wi = (const float*)a.Wi + wrow;
      const float* wf = (const float*)a.Wf + wrow;
      const float* wr = (const float*)a.Wr + wrow;
      f32x4 ci = {0.f, 0.f, 0.f, 0.f}, cf = ci, cr = ci;

      for (int k0 = 0; k0 < a.GH; k0 += 16) {
        const int kk = k0 + g * 4;
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 av = t_ok ? *reinterpret_cast<const float4*>(Arow + kk) : z;
        float4 bv = ok ? *reinterpret_cast<const float4*>(Brow + kk) : z;
        float4 vi = n_ok ? *reinterpret_cast<const float4*>(wi + kk) : z;
        float4 vf = n_ok ? *reinterpret_cast<const float4*>(wf + kk) : z;
        float4 vr = n_ok ? *reinterpret_cast<const float4*>(wr + kk) : z;
        const float ha[4] = {av.x + bv.x, av.y + bv.y, av.z + bv.z, av.w + bv.w};
        const float wia[4] = {vi.x, vi.y, vi.z, vi.w};
        const float wfa[4] = {vf.x, vf.y, vf.z, vf.w};
        const float wra[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float x = fmaxf(ha[j], 0.f);
          x = x * x;
          ci = __builtin_amdgcn_mfma_f32_16x16x4f32(x, wia[j], ci, 0, 0, 0);
          cf = __builtin_amdgcn_mfma_f32_16x16x4f32(x, wfa[j], cf, 0, 0, 0);
          cr = __builtin_amdgcn_mfma_f32_16x16x4f32(x, wra[j], cr, 0, 0, 0);
        }
      }
      if (n_ok) {
        const float bvi = a.bi[l * a.H + n], bvf = a.bf[l * a.H + n], bvr = a.br[l * a.H + n];
        const int tb = blockIdx.x * kTileT + wave * 16 + g * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int to = tb + i;
          if (to < a.T) {
            const int64_t o = (((int64_t)b * a.T + to) * a.n_lv + l) * a.H + n;
            ((float*)a.oi)[o] = ci[i] + bvi;
            ((float*)a.of)[o] = cf[i] + bvf;
            ((float*)a.orr)[o] = cr[i] + bvr;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// backward (reference dispatcher_hybrid/fused_gates.py:96-173)
//   dh[t,l,k]  = sum_{x,h} dP_x[t,l,h] * W_x[l,h,k]
//   dx[t,l,k]  = 2 * relu(a + ok*b)[k] * dh[t,l,k]        (a+b rounded as in the forward)
//   dA[t]      = sum_l dx[t,l]                   -- summed in registers, one writer per element
//   dB[t-2^l] += ok * dx[t,l]                    -- fp32 atomics (levels collide)
//   dW_x[l,h] += sum_t hid[t,l] * dP_x[t,l,h]    -- fp32 atomics across tiles
//   db_x[l,h] += sum_t dP_x[t,l,h]               -- fp32 atomics across tiles
// One workgroup per (batch row, 64-position tile), one thread per (position, k-chunk). Plain fp32
// FMA: the backward is off the measured paths.
// ---------------------------------------------------------------------------------------------
struct BwdArgs {
  const void* A;
  const void* B;
  int64_t sab, sat;
  const void* Wi;
  const void* Wf;
  const void* Wr;
  int64_t swl, swh;
  const void* dPi;
  const void* dPf;
  const void* dPr;
  const void* mask;
  int64_t smb, smt;
  float* dA;
  float* dB;
  float* dWi;
  float* dWf;
  float* dWr;
  float* dbi;
  float* dbf;
  float* dbr;
  int b, T, GH, H, n_lv;
};

__global__ void fill_zero(float* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

constexpr int kBwdTile = 16;   // positions per workgroup
constexpr int kBwdMaxH = 64;

template <typename T>
__global__ __launch_bounds__(kThreads) void gate_preacts_bwd_kernel(BwdArgs a) {
  __shared__ float dp[3][kBwdTile][kBwdMaxH];
  __shared__ int okm[kBwdTile];
  const int b = blockIdx.y;
  const int t0 = blockIdx.x * kBwdTile;
  const int tid = threadIdx.x;
  const T* Ab = (const T*)a.A + (int64_t)b * a.sab;
  const T* Bb = (const T*)a.B + (int64_t)b * a.sab;
  const bool is_bf16 = sizeof(T) == 2;

  // dA accumulator: thread owns k = tid, tid + 256, ... for every position of the tile (GH <= 4096)
  for (int k = tid; k < a.GH; k += kThreads)
    for (int i = 0; i < kBwdTile; ++i)
      if (t0 + i < a.T) a.dA[((int64_t)b * a.T + t0 + i) * a.GH + k] = 0.f;
  __syncthreads();

  for (int l = 0; l < a.n_lv; ++l) {
    // stage dP for the tile's positions at this level
    for (int e = tid; e < 3 * kBwdTile * a.H; e += kThreads) {
      const int x = e / (kBwdTile * a.H), rem = e % (kBwdTile * a.H), i = rem / a.H, h = rem % a.H;
      const int t = t0 + i;
      float v = 0.f;
      if (t < a.T) {
        const T* src = (const T*)(x == 0 ? a.dPi : x == 1 ? a.dPf : a.dPr);
        v = Elem<T>::load(src + (((int64_t)b * a.T + t) * a.n_lv + l) * a.H + h);
      }
      dp[x][i][h] = v;
    }
    if (tid < kBwdTile) {
      const int t = t0 + tid;
      int ok = t < a.T && t >= (1 << l);
      if (ok && a.mask) ok = Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)t * a.smt + l) > 0.f;
      okm[tid] = ok;
    }
    __syncthreads();
    // bias gradients: thread per (gate, head)
    if (tid < 3 * a.H) {
      const int x = tid / a.H, h = tid % a.H;
      float s = 0.f;
      for (int i = 0; i < kBwdTile; ++i) s += dp[x][i][h];
      float* db = x == 0 ? a.dbi : x == 1 ? a.dbf : a.dbr;
      atomicAdd(db + l * a.H + h, s);
    }
    for (int k = tid; k < a.GH; k += kThreads) {
      for (int i = 0; i < kBwdTile; ++i) {
        const int t = t0 + i;
        if (t >= a.T) break;
        const bool ok = okm[i];
        const float av = Elem<T>::load(Ab + (int64_t)t * a.sat + k);
        const float bv = ok ? Elem<T>::load(Bb + (int64_t)(t - (1 << l)) * a.sat + k) : 0.f;
        float x = av + bv;
        if (is_bf16) x = Elem<T>::round(x);
        const float rx = fmaxf(x, 0.f);
        const float hid = Elem<T>::round(rx * rx);
        float dh = 0.f;
        for (int h = 0; h < a.H; ++h) {
          const int64_t w = (int64_t)l * a.swl + (int64_t)h * a.swh + k;
          dh += dp[0][i][h] * Elem<T>::load((const T*)a.Wi + w) + dp[1][i][h] * Elem<T>::load((const T*)a.Wf + w) +
                dp[2][i][h] * Elem<T>::load((const T*)a.Wr + w);
        }
        const float dx = 2.f * rx * dh;
        a.dA[((int64_t)b * a.T + t) * a.GH + k] += dx;
        if (ok) atomicAdd(a.dB + ((int64_t)b * a.T + (t - (1 << l))) * a.GH + k, dx);
      }
      // weight gradients for this k over the tile
      for (int h = 0; h < a.H; ++h) {
        float si = 0.f, sf = 0.f, sr = 0.f;
        for (int i = 0; i < kBwdTile; ++i) {
          const int t = t0 + i;
          if (t >= a.T) break;
          const bool ok = okm[i];
          const float av = Elem<T>::load(Ab + (int64_t)t * a.sat + k);
          const float bv = ok ? Elem<T>::load(Bb + (int64_t)(t - (1 << l)) * a.sat + k) : 0.f;
          float x = av + bv;
          if (is_bf16) x = Elem<T>::round(x);
          const float rx = fmaxf(x, 0.f);
          const float hid = Elem<T>::round(rx * rx);
          si += hid * dp[0][i][h];
          sf += hid * dp[1][i][h];
          sr += hid * dp[2][i][h];
        }
        const int64_t w = ((int64_t)l * a.H + h) * a.GH + k;
        atomicAdd(a.dWi + w, si);
        atomicAdd(a.dWf + w, sf);
        atomicAdd(a.dWr + w, sr);
      }
    }
    __syncthreads();
  }
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; }

int check_shapes(const char* who, int dtype, int b, int T, int GH, int H, int n_lv) {
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(b >= 1 && T >= 1, DH_ERR_INVALID_ARG, "%s: b=%d T=%d must be >= 1", who, b, T);
  DH_REQUIRE(GH >= 64 && GH % 64 == 0, DH_ERR_UNSUPPORTED_SHAPE, "%s: GH=%d not a multiple of 64", who, GH);
  DH_REQUIRE(H >= 1 && H <= 64, DH_ERR_UNSUPPORTED_SHAPE, "%s: H=%d not in [1,64]", who, H);
  DH_REQUIRE(n_lv >= 1 && n_lv <= 16, DH_ERR_UNSUPPORTED_SHAPE, "%s: n_lv=%d not in [1,16]", who, n_lv);
  DH_REQUIRE(T <= (1 << 30) / 4, DH_ERR_UNSUPPORTED_SHAPE, "%s: T=%d too large", who, T);
  return DH_OK;
}

}  // namespace

extern "C" int dh_gate_preacts_fwd(int dtype, const void* A, const void* B, int64_t stride_ab, int64_t stride_at,
                                   const void* Wi, const void* Wf, const void* Wr, int64_t stride_wl,
                                   int64_t stride_wh, const float* bi, const float* bf, const float* br,
                                   const void* mask, int64_t stride_mb, int64_t stride_mt, void* out_i,
                                   void* out_f, void* out_r, int b, int T, int GH, int H, int n_lv,
                                   void* stream) {
  const char* who = "dh_gate_preacts_fwd";
  int st = check_shapes(who, dtype, b, T, GH, H, n_lv);
  if (st) return st;
  DH_REQUIRE(A && B && Wi && Wf && Wr && bi && bf && br && out_i && out_f && out_r, DH_ERR_INVALID_ARG,
             "%s: null pointer argument", who);
  const int vec = dtype == DH_BF16 ? 8 : 4;  // elements per 16-byte load
  DH_REQUIRE(aligned(A, 16) && aligned(B, 16) && aligned(Wi, 16) && aligned(Wf, 16) && aligned(Wr, 16) &&
                 stride_at % vec == 0 && stride_ab % vec == 0 && stride_wl % vec == 0 && stride_wh % vec == 0,
             DH_ERR_INVALID_ARG, "%s: A/B/W rows need 16-byte alignment", who);
  DH_REQUIRE(stride_at >= GH && stride_wh >= GH && stride_wl >= (int64_t)H * stride_wh, DH_ERR_INVALID_ARG,
             "%s: strides overlap rows", who);
  FwdArgs a{A, B, stride_ab, stride_at, Wi, Wf, Wr, stride_wl, stride_wh, bi, bf, br, mask, stride_mb, stride_mt,
            out_i, out_f, out_r, b, T, GH, H, n_lv};
  dim3 grid((T + kTileT - 1) / kTileT, b), block(kThreads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_BF16)
    gate_preacts_fwd_bf16<<<grid, block, 0, s>>>(a);
  else
    gate_preacts_fwd_f32<<<grid, block, 0, s>>>(a);
  return dh_check_launch(who);
}

extern "C" int dh_gate_preacts_bwd(int dtype, const void* A, const void* B, int64_t stride_ab, int64_t stride_at,
                                   const void* Wi, const void* Wf, const void* Wr, int64_t stride_wl,
                                   int64_t stride_wh, const void* dPi, const void* dPf, const void* dPr,
                                   const void* mask, int64_t stride_mb, int64_t stride_mt, float* dA, float* dB,
                                   float* dWi, float* dWf, float* dWr, float* dbi, float* dbf, float* dbr, int b,
                                   int T, int GH, int H, int n_lv, void* stream) {
  const char* who = "dh_gate_preacts_bwd";
  int st = check_shapes(who, dtype, b, T, GH, H, n_lv);
  if (st) return st;
  DH_REQUIRE(A && B && Wi && Wf && Wr && dPi && dPf && dPr && dA && dB && dWi && dWf && dWr && dbi && dbf && dbr,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  hipStream_t s = (hipStream_t)stream;
  BwdArgs a{A, B, stride_ab, stride_at, Wi, Wf, Wr, stride_wl, stride_wh, dPi, dPf, dPr, mask, stride_mb,
            stride_mt, dA, dB, dWi, dWf, dWr, dbi, dbf, dbr, b, T, GH, H, n_lv};
  const int64_t nAB = (int64_t)b * T * GH, nW = (int64_t)n_lv * H * GH, nb = (int64_t)n_lv * H;
  fill_zero<<<1024, 256, 0, s>>>(dB, nAB);
  for (float* p : {dWi, dWf, dWr}) fill_zero<<<256, 256, 0, s>>>(p, nW);
  for (float* p : {dbi, dbf, dbr}) fill_zero<<<1, 256, 0, s>>>(p, nb);
  st = dh_check_launch(who);
  if (st) return st;
  dim3 grid((T + kBwdTile - 1) / kBwdTile, b), block(kThreads);
  if (dtype == DH_BF16)
    gate_preacts_bwd_kernel<bf16_t><<<grid, block, 0, s>>>(a);
  else
    gate_preacts_bwd_kernel<float><<<grid, block, 0, s>>>(a);
  return dh_check_launch(who);
}
