// Parallel gate pre-activations (and their backward) for gfx950.
//
// Forward semantics (reference dispatcher_hybrid/fused_gates.py:38-93 and the eager definition at
// dispatcher_hybrid/modeling_dispatcher.py:100-109):
//   ok[b,t,l]      = t < T && t >= 2^l && (mask == null || mask[b,t,l] > 0)
//   hid[b,t,l,k]   = relu(A[b,t,k] + ok * B[b,t-2^l,k])^2
//   pre_x[b,t,l,h] = sum_k hid[b,t,l,k] * W_x[l,h,k] + b_x[l,h]          x in {i, f, r}
// bf16 mode rounds a+b and hid to bf16 (the points where the eager bf16 path rounds; the hardware
// v_cvt_pk_bf16_f32 rounds to nearest even), multiplies on bf16 MFMA with fp32 accumulation, adds
// the fp32 bias and rounds once on store. fp32 mode uses fp32 MFMA throughout. The outputs are
// written through element strides, so a caller can ask for the (b, T, n_lv, H) layout of the
// reference op or for the head-major (b, H, n_lv, T) layout the level scan reads best.
//
// Work decomposition: one workgroup (4 wave64s) per (64-position tile, group of LG levels, batch
// row); wave w owns positions 16w..16w+15 of the tile. For each k-chunk the lane's A fragment is
// loaded once and reused by all LG levels of the group; each level adds its lagged B fragment,
// forms the hidden tile in MFMA A-operand registers (lane -> row lane%16, k-chunk lane/16) and
// multiplies it against W_x[l] (B operand: lane -> head lane%16) for the three gates, N = 16 heads
// per MFMA tile. The k-loop is software-pipelined: the fragments of step k+1 are requested before
// the MFMAs of step k are issued. The host picks LG so that tiles x groups fills the chip (small
// prefills get one level per workgroup, long ones reuse A over four) and KU, the k-chunks per step,
// so every step keeps enough bytes in flight.
#include "dh_common.h"

#include <utility>

namespace {

constexpr int kThreads = 256;
constexpr int kTileT = 64;

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

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
  int64_t smb, smt, sml;
  void* oi;
  void* of;
  void* orr;
  int64_t sob, sot, sol, soh;
  int b, T, GH, H, n_lv;
  int vec_out;                  // outputs take 4-position vector stores (head-major, aligned)
  int activate;                 // write the scan's gates a, f, r instead of pre-activations
};

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Raw buffer access: a descriptor (base, byte range) held in scalar registers, a per-lane byte
// offset (voffset) and a uniform byte offset (soffset); no per-lane 64-bit address arithmetic, and
// a read past the range returns zeros. dword3 = 0x00020000 is the gfx9-family raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// two fp32 -> packed bf16 (round to nearest even, hardware conversion)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// bf16-valued fp32 from fp32 in ONE instruction: v_cvt_pk_bf16_f32(0, x) puts bf16(x) in the high
// half and bf16(0) = 0 in the low half, which are exactly the fp32 bits of the rounded value
// (written as the instruction itself: the compiler otherwise converts into the low half and then
// permutes, two instructions). PRECONDITION: x must not come straight from a transcendental
// instruction (v_exp/v_rcp/...): gfx950 needs a wait state before a VALU reads a transcendental
// result and the compiler's hazard pass does not look into inline assembly. The hot loop feeds it
// v_max results only; everything else rounds with round_bf16_sw.
__device__ __forceinline__ float round_bf16_sw(float x) { return bf16_to_f32(f32_to_bf16(x)); }
// the same through the compiler's own conversion (v_cvt_pk_bf16_f32 + shift; round to nearest
// even, NaN stays NaN), usable on transcendental results
__device__ __forceinline__ float round_bf16_cc(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ float round_bf16(float x) {
  float r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
  return r;
}

// Element math of the two modes. KC = k elements one 16-byte fragment per lane covers across the
// wave's four lane groups. unpack_a converts the A fragment once per k-step (shared by every level
// of the group); mma3 adds hid(a, b) . W_x for the three gates of one level. A masked row's B
// fragment arrives as zeros (out-of-range buffer read), so no masking happens here.
struct MathBf16 {
  typedef bf16_t T;
  static constexpr int KC = 32;
  static constexpr int KL = 8;      // k elements per lane fragment
  __device__ __forceinline__ static void unpack_a(const uint4& av, float (&af)[8]) {
    const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      af[2 * j] = __uint_as_float(aw[j] << 16);
      af[2 * j + 1] = __uint_as_float(aw[j] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void mma3(f32x4 (&acc)[3], const float (&af)[8], const uint4& bv,
                                              const uint4 (&w)[3]) {
    const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
    uint32_t hw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // relu(round(a+b)) = round(relu(a+b)); its square is exact in fp32 and rounded once
      const float x0 = round_bf16(fmaxf(af[2 * j] + __uint_as_float(bw[j] << 16), 0.f));
      const float x1 = round_bf16(fmaxf(af[2 * j + 1] + __uint_as_float(bw[j] & 0xffff0000u), 0.f));
      hw[j] = pack_bf16x2(x0 * x0, x1 * x1);
    }
    bf16x8 hid, wi, wf, wr;
    __builtin_memcpy(&hid, hw, 16);
    __builtin_memcpy(&wi, &w[0], 16);
    __builtin_memcpy(&wf, &w[1], 16);
    __builtin_memcpy(&wr, &w[2], 16);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hid, wi, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hid, wf, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hid, wr, acc[2], 0, 0, 0);
  }
  __device__ __forceinline__ static T out(float v) { return f32_to_bf16(v); }
  __device__ __forceinline__ static float rnd(float v) { return round_bf16_sw(v); }
  __device__ __forceinline__ static void store4(T* p, const float (&v)[4]) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  }
};

// fp32: 16x16x4 fp32 MFMA; lane group g holds k = 4g..4g+3 of the 16-wide chunk and issues 4 MFMAs
// per gate, MFMA j taking k = 4g + j on both operands.
struct MathF32 {
  typedef float T;
  static constexpr int KC = 16;
  static constexpr int KL = 4;
  __device__ __forceinline__ static void unpack_a(const uint4& av, float (&af)[4]) {
    af[0] = __uint_as_float(av.x);
    af[1] = __uint_as_float(av.y);
    af[2] = __uint_as_float(av.z);
    af[3] = __uint_as_float(av.w);
  }
  __device__ __forceinline__ static void mma3(f32x4 (&acc)[3], const float (&af)[4], const uint4& bv,
                                              const uint4 (&w)[3]) {
    const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
    const uint32_t wi[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
    const uint32_t wf[4] = {w[1].x, w[1].y, w[1].z, w[1].w};
    const uint32_t wr[4] = {w[2].x, w[2].y, w[2].z, w[2].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x = fmaxf(af[j] + __uint_as_float(bw[j]), 0.f);
      x = x * x;
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, __uint_as_float(wi[j]), acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, __uint_as_float(wf[j]), acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, __uint_as_float(wr[j]), acc[2], 0, 0, 0);
    }
  }
  __device__ __forceinline__ static T out(float v) { return v; }
  __device__ __forceinline__ static float rnd(float v) { return v; }
  __device__ __forceinline__ static void store4(T* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

template <typename M, int LG, int KU, bool HAS_MASK>
__global__ __launch_bounds__(kThreads) void gate_preacts_fwd_kernel(FwdArgs a) {
  typedef typename M::T T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int b = blockIdx.z;
  const int l0 = blockIdx.y * LG;
  const int t = blockIdx.x * kTileT + wave * 16 + r;   // row this lane feeds into the MFMA
  const bool t_ok = t < a.T;
  const int tc = t_ok ? t : a.T - 1;
  // addresses: workgroup-uniform base pointers plus per-lane 32-bit byte offsets (the host checks
  // they fit), so every load is one scalar-base + vector-offset access with no 64-bit arithmetic
  const uint32_t row_bytes = (uint32_t)((int64_t)a.T * a.sat * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rA = buf_rsrc((const T*)a.A + (int64_t)b * a.sab, row_bytes);
  const __amdgpu_buffer_rsrc_t rB = buf_rsrc((const T*)a.B + (int64_t)b * a.sab, row_bytes);
  const uint32_t aoff = (uint32_t)(((int64_t)tc * a.sat + g * M::KL) * (int64_t)sizeof(T));

  int lv[LG];
  uint32_t boff[LG];
  float mv[LG];
#pragma unroll
  for (int j = 0; j < LG; ++j) {
    lv[j] = min(l0 + j, a.n_lv - 1);
    mv[j] = 1.f;
    if (HAS_MASK)
      mv[j] = Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)tc * a.smt + (int64_t)lv[j] * a.sml);
  }
#pragma unroll
  for (int j = 0; j < LG; ++j) {
    const int src = tc - (1 << lv[j]);             // rows past T use the clamped row: always < T
    const bool keep = t_ok && src >= 0 && l0 + j < a.n_lv && mv[j] > 0.f;
    // a row without a source reads past the descriptor's range, which returns zeros (B = 0)
    boff[j] = keep ? (uint32_t)(((int64_t)src * a.sat + g * M::KL) * (int64_t)sizeof(T)) : 0x80000000u;
  }

  const int NT = (a.H + 15) >> 4;
  constexpr int STEP = M::KC * KU;
  for (int nt = 0; nt < NT; ++nt) {
    const int n = nt * 16 + r;                  // head whose weights this lane feeds
    const int nc = n < a.H ? n : a.H - 1;
    const uint32_t woff = (uint32_t)(((int64_t)nc * a.swh + g * M::KL) * (int64_t)sizeof(T));
    const uint32_t w_bytes = (uint32_t)((int64_t)a.n_lv * a.swl * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t rW[3] = {buf_rsrc(a.Wi, w_bytes), buf_rsrc(a.Wf, w_bytes), buf_rsrc(a.Wr, w_bytes)};
    uint32_t wlo[LG];
#pragma unroll
    for (int j = 0; j < LG; ++j) wlo[j] = (uint32_t)((int64_t)lv[j] * a.swl * (int64_t)sizeof(T));
    f32x4 acc[LG][3];
#pragma unroll
    for (int j = 0; j < LG; ++j)
#pragma unroll
      for (int x = 0; x < 3; ++x) acc[j][x] = f32x4{0.f, 0.f, 0.f, 0.f};

    // two fragment buffers in ping-pong (no register copies, so a prefetch is never waited for
    // before the MFMAs of the other buffer have been issued). The host makes GH a multiple of
    // 2*STEP, so both halves of every iteration are real work (no branch the loads could sink
    // into); the fetch after the last step is clamped to a valid chunk and never used.
    uint4 xA[KU], xB[KU][LG], xW[KU][LG][3];
    uint4 yA[KU], yB[KU][LG], yW[KU][LG][3];
    auto fetch = [&](int k0, uint4 (&fA)[KU], uint4 (&fB)[KU][LG], uint4 (&fW)[KU][LG][3]) {
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const uint32_t kb = (uint32_t)((k0 + u * M::KC) * (int)sizeof(T));   // uniform byte offset
        fA[u] = bld16(rA, aoff, kb);
#pragma unroll
        for (int j = 0; j < LG; ++j) fB[u][j] = bld16(rB, boff[j], kb);
#pragma unroll
        for (int j = 0; j < LG; ++j)
#pragma unroll
          for (int x = 0; x < 3; ++x) fW[u][j][x] = bld16(rW[x], woff, wlo[j] + kb);
      }
    };
    auto compute = [&](const uint4 (&fA)[KU], const uint4 (&fB)[KU][LG], const uint4 (&fW)[KU][LG][3]) {
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        float af[M::KL];
        M::unpack_a(fA[u], af);
#pragma unroll
        for (int j = 0; j < LG; ++j) M::mma3(acc[j], af, fB[u][j], fW[u][j]);
      }
    };
    fetch(0, xA, xB, xW);
    for (int k0 = 0; k0 < a.GH; k0 += 2 * STEP) {
      fetch(k0 + STEP, yA, yB, yW);
      compute(xA, xB, xW);
      fetch(k0 + 2 * STEP < a.GH ? k0 + 2 * STEP : k0, xA, xB, xW);
      compute(yA, yB, yW);
    }
    // C fragment: column (head) lane%16, rows 4*(lane/16) + i
    const int tb = blockIdx.x * kTileT + wave * 16 + g * 4;
    const bool vec = a.vec_out && tb + 3 < a.T;
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int l = l0 + j;
      if (l >= a.n_lv || n >= a.H) continue;
      const float bias[3] = {a.bi[l * a.H + n], a.bf[l * a.H + n], a.br[l * a.H + n]};
      T* outs[3] = {(T*)a.oi, (T*)a.of, (T*)a.orr};
      const int64_t base = (int64_t)b * a.sob + (int64_t)l * a.sol + (int64_t)n * a.soh;
      float v[3][4];
#pragma unroll
      for (int x = 0; x < 3; ++x)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[x][i] = acc[j][x][i] + bias[x];
      if (a.activate) {
        // a = sigmoid(pre_i) * M, f = sigmoid(pre_f) * M + 1 - M, r = sigmoid(pre_r), rounded where
        // the eager bf16 path rounds (pre-activation, sigmoid output); M = [t >= 2^l] * [mask > 0]
        float mval[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mval[i] = 1.f;
          if (HAS_MASK) {
            const int to = min(tb + i, a.T - 1);
            mval[i] = Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)to * a.smt + (int64_t)l * a.sml);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float m = (tb + i >= (1 << l) && mval[i] > 0.f) ? 1.f : 0.f;
          const float si = M::rnd(dh_sigmoid(M::rnd(v[0][i])));
          const float sf = M::rnd(dh_sigmoid(M::rnd(v[1][i])));
          const float sr = M::rnd(dh_sigmoid(M::rnd(v[2][i])));
          v[0][i] = si * m;
          v[1][i] = sf * m + (1.f - m);
          v[2][i] = sr;
        }
      }
#pragma unroll
      for (int x = 0; x < 3; ++x) {
        if (vec) {
          M::store4(outs[x] + base + tb, v[x]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (tb + i < a.T) outs[x][base + (int64_t)(tb + i) * a.sot] = M::out(v[x][i]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// bf16 forward with the weights staged in LDS (H <= 16).
//
// The kernel above streams every weight fragment from the cache hierarchy into every wave: per
// k-step a wave reads 3 KB of weights per level for 1 KB of activations, and at C5 sizes
// (b = 8, T = 4096) the launch is bound by those cache reads (L2 requests ~25x the bytes the
// launch needs) and by the waits on them. Here a workgroup of 4 waves owns P = 64*MB positions and
// LG levels; for each 64-wide k-chunk it copies the chunk of W_i/W_f/W_r of its levels
// (LG x 3 x 16 heads x 64 k, bf16) into LDS once, with rows padded to 144 bytes so the 16-byte
// reads of the MFMA B operand (lanes = 16 heads x 4 k-groups) hit distinct banks, and every wave
// reads each fragment once for its MB row blocks of 16 positions. The activation fragments (A
// rows, lagged B rows) go straight from memory into MFMA A-operand registers, one k-step ahead;
// the next chunk's weights are requested at the start of a chunk and written to the other LDS
// buffer at its end (one barrier per chunk). Same arithmetic, rounding points and outputs as the
// kernel above.
// ---------------------------------------------------------------------------------------------
// Register sets of the one-level kernel's prefetch: chunks requested two ahead. Measured on MI355X
// (activated readouts + scan per layer, b = 1, us at T = 1024 / 2048 / 3840): three sets 22.4 /
// 32.3 / 45.8, four 22.2 / 32.3 / 46.8, five 22.3 / 32.4 / 47.2 (six spill at the occupancy the
// launch bounds ask for).
constexpr int kSets = 3;
static_assert(kSets >= 2, "at least the chunk computed and the one in flight");
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<0>) ... f(integral_constant<N - 1>), unrolled with compile-time indices
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
constexpr int kLdsKC = 64;                      // k elements per LDS weight chunk (2 MFMA k-steps)
constexpr int kLdsRow = kLdsKC * 2 + 16;         // padded LDS row: 144 bytes

// occupancy by register footprint: (levels x row blocks) accumulators plus two chunks of fragments
template <int LG, int MB> struct LdsOcc { static constexpr int value = LG * MB >= 4 ? 2 : 3; };

template <int LG, int MB, bool HAS_MASK>
__global__ __launch_bounds__(kThreads, (LdsOcc<LG, MB>::value)) void gate_preacts_fwd_lds_kernel(FwdArgs a) {
  typedef bf16_t T;
  constexpr int P = 64 * MB;                     // positions per workgroup
  constexpr int WBYTES = LG * 3 * 16 * kLdsRow;  // one LDS weight buffer
  constexpr int PIECES = LG * 3 * 16 * (kLdsKC / 8);   // 16-byte pieces of one chunk
  constexpr int PPT = (PIECES + kThreads - 1) / kThreads;
  __shared__ __align__(16) unsigned char wl[2][WBYTES];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int b = blockIdx.z;
  const int l0 = blockIdx.y * LG;
  const int tbase = blockIdx.x * P + wave * 16 * MB;   // first position of the wave

  const uint32_t row_bytes = (uint32_t)((int64_t)a.T * a.sat * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rA = buf_rsrc((const T*)a.A + (int64_t)b * a.sab, row_bytes);
  const __amdgpu_buffer_rsrc_t rB = buf_rsrc((const T*)a.B + (int64_t)b * a.sab, row_bytes);
  const uint32_t w_bytes = (uint32_t)((int64_t)a.n_lv * a.swl * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rW[3] = {buf_rsrc(a.Wi, w_bytes), buf_rsrc(a.Wf, w_bytes), buf_rsrc(a.Wr, w_bytes)};

  // ---- activation loads. The MFMA A operand wants lane (r, g) = (lane % 16, lane / 16) to hold
  // 16 bytes of row r; loaded that way, the four lanes of every quad read four different rows and
  // the texture unit serves the load at a quarter of its rate (measured: the data return path busy
  // ~80% of the launch). So lane S loads piece S & 3 of row S >> 2 (each quad reads 64 contiguous
  // bytes of one row) and four ds_bpermute moves per fragment hand lane (r, g) the piece of source
  // lane 4 r + g.
  const int crow = lane >> 2, cpiece = lane & 3;
  const int bperm = 4 * (4 * r + g);                 // byte address of the source lane
  uint32_t aoff[MB], boff[MB][LG];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int t = tbase + 16 * mb + crow;
    const bool t_ok = t < a.T;
    const int tc = t_ok ? t : a.T - 1;
    aoff[mb] = (uint32_t)(((int64_t)tc * a.sat + cpiece * 8) * (int64_t)sizeof(T));
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int lv = min(l0 + j, a.n_lv - 1);
      float mv = 1.f;
      if (HAS_MASK)
        mv = Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)tc * a.smt + (int64_t)lv * a.sml);
      const int src = tc - (1 << lv);
      const bool keep = t_ok && src >= 0 && l0 + j < a.n_lv && mv > 0.f;
      // a row without a source reads past the descriptor's range, which returns zeros (B = 0)
      boff[mb][j] = keep ? (uint32_t)(((int64_t)src * a.sat + cpiece * 8) * (int64_t)sizeof(T)) : 0x80000000u;
    }
  }
  auto to_mfma = [&](const uint4& v) {
    return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(bperm, (int)v.x),
                      (uint32_t)__builtin_amdgcn_ds_bpermute(bperm, (int)v.y),
                      (uint32_t)__builtin_amdgcn_ds_bpermute(bperm, (int)v.z),
                      (uint32_t)__builtin_amdgcn_ds_bpermute(bperm, (int)v.w));
  };

  // ---- weight chunk copy: piece q = tid + 256 i -> (level j, gate x, head n, 16-byte column c).
  // A (level, gate) block is 16 rows x 8 pieces = 128 pieces = two waves, so the block index
  // jx = q >> 7 = 2 i + wave / 2 is uniform over a wave: its descriptor is picked with scalar
  // selects (a per-lane descriptor would make the compiler loop over the lanes' distinct values).
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  uint32_t wsrc[PPT], wdst[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int q = min(tid + i * kThreads, PIECES - 1);
    const int c = q & 7, n = (q >> 3) & 15;
    const int jx = min(2 * i + (wave_u >> 1), 3 * LG - 1);   // = q >> 7 (uniform)
    const int j = jx / 3;
    const int lv = min(l0 + j, a.n_lv - 1), nc = min(n, a.H - 1);
    wsrc[i] = (uint32_t)(((int64_t)lv * a.swl + (int64_t)nc * a.swh + c * 8) * (int64_t)sizeof(T));
    wdst[i] = (uint32_t)((jx * 16 + n) * kLdsRow + c * 16);
  }
  uint4 wst[PPT];
  auto w_fetch = [&](int k0) {
    const uint32_t kb = (uint32_t)(k0 * (int)sizeof(T));
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int jx = min(2 * i + (wave_u >> 1), 3 * LG - 1);
      const int x = jx % 3;
      const __amdgpu_buffer_rsrc_t rw = x == 0 ? rW[0] : (x == 1 ? rW[1] : rW[2]);
      wst[i] = bld16(rw, wsrc[i], kb);
    }
  };
  auto w_store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PPT; ++i)
      if (tid + i * kThreads < PIECES) *reinterpret_cast<uint4*>(&wl[buf][wdst[i]]) = wst[i];
  };

  f32x4 acc[MB][LG][3];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < LG; ++j)
#pragma unroll
      for (int x = 0; x < 3; ++x) acc[mb][j][x] = f32x4{0.f, 0.f, 0.f, 0.f};

  // activation fragments of one chunk (2 k-steps): A rows and the LG lagged B rows of each row
  // block. Two chunk buffers in ping-pong: the next chunk's fragments are in flight during the
  // whole current chunk (the loads' latency under load is several k-steps of arithmetic).
  uint4 xA[2][MB], xB[2][MB][LG], yA[2][MB], yB[2][MB][LG];
  auto fetch = [&](int k0, uint4 (&fA)[2][MB], uint4 (&fB)[2][MB][LG]) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint32_t kb = (uint32_t)((k0 + 32 * kk) * (int)sizeof(T));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        fA[kk][mb] = bld16(rA, aoff[mb], kb);
#pragma unroll
        for (int j = 0; j < LG; ++j) fB[kk][mb][j] = bld16(rB, boff[mb][j], kb);
      }
    }
  };
  // one chunk from the LDS weight buffer `buf`
  auto compute = [&](const uint4 (&fA)[2][MB], const uint4 (&fB)[2][MB][LG], int buf) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      float af[MB][8];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) MathBf16::unpack_a(to_mfma(fA[kk][mb]), af[mb]);
#pragma unroll
      for (int j = 0; j < LG; ++j) {
        uint4 w[3];
#pragma unroll
        for (int x = 0; x < 3; ++x)
          w[x] = *reinterpret_cast<const uint4*>(&wl[buf][((j * 3 + x) * 16 + r) * kLdsRow + kk * 64 + g * 16]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) MathBf16::mma3(acc[mb][j], af[mb], to_mfma(fB[kk][mb][j]), w);
      }
    }
  };
  const int nchunk_ = a.GH / kLdsKC;
  // chunk c: request chunk c+1 (weights and fragments), compute chunk c, store the weights of c+1
  auto chunk = [&](int c, const uint4 (&cA)[2][MB], const uint4 (&cB)[2][MB][LG], uint4 (&nA)[2][MB],
                   uint4 (&nB)[2][MB][LG]) {
    const bool more = c + 1 < nchunk_;                   // uniform
    if (more) {
      w_fetch((c + 1) * kLdsKC);
      fetch((c + 1) * kLdsKC, nA, nB);
    }
    compute(cA, cB, c & 1);
    if (more) w_store((c + 1) & 1);
    __syncthreads();
  };

  if constexpr (LG == 1) {
    // One-level tiles (short prefills: one workgroup per CU, nothing else to hide a round trip):
    // weights and fragments are requested kSets - 1 chunks ahead, in kSets register sets each, so
    // neither the compute of chunk c nor the LDS write of c+1's weights waits on a load issued in
    // the last kSets - 2 chunks. Chunk c computes from set c % kSets, requests chunk c + kSets - 1
    // into the set chunk c - 1 used, and writes the weights of chunk c + 1 to LDS.
    constexpr int NS = kSets;
    uint4 sA[NS][2][MB], sB[NS][2][MB][LG], sW[NS][PPT];
    auto w_fetch3 = [&](int k0, uint4 (&ws)[PPT]) {
      const uint32_t kb = (uint32_t)(k0 * (int)sizeof(T));
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int jx = min(2 * i + (wave_u >> 1), 3 * LG - 1);
        const int x = jx % 3;
        const __amdgpu_buffer_rsrc_t rw = x == 0 ? rW[0] : (x == 1 ? rW[1] : rW[2]);
        ws[i] = bld16(rw, wsrc[i], kb);
      }
    };
    auto w_store3 = [&](int buf, const uint4 (&ws)[PPT]) {
#pragma unroll
      for (int i = 0; i < PPT; ++i)
        if (tid + i * kThreads < PIECES) *reinterpret_cast<uint4*>(&wl[buf][wdst[i]]) = ws[i];
    };
    auto step = [&](int c, auto uc) {
      constexpr int u = decltype(uc)::value;             // c % NS
      constexpr int uf = (u + NS - 1) % NS, un = (u + 1) % NS;
      if (c + NS - 1 < nchunk_) {                        // uniform
        w_fetch3((c + NS - 1) * kLdsKC, sW[uf]);
        fetch((c + NS - 1) * kLdsKC, sA[uf], sB[uf]);
      }
      compute(sA[u], sB[u], c & 1);
      if (c + 1 < nchunk_) w_store3((c + 1) & 1, sW[un]);
      __syncthreads();
    };
    static_for<NS - 1>([&](auto uc) {
      constexpr int u = decltype(uc)::value;
      if (u < nchunk_) {
        w_fetch3(u * kLdsKC, sW[u]);
        fetch(u * kLdsKC, sA[u], sB[u]);
      }
    });
    w_store3(0, sW[0]);
    __syncthreads();
    int c = 0;
    for (; c + NS - 1 < nchunk_; c += NS) static_for<NS>([&](auto uc) { step(c + decltype(uc)::value, uc); });
    static_for<NS - 1>([&](auto uc) {
      if (c + decltype(uc)::value < nchunk_) step(c + decltype(uc)::value, uc);
    });
  } else {
    w_fetch(0);
    fetch(0, xA, xB);
    w_store(0);
    __syncthreads();
    int c = 0;
    for (; c + 1 < nchunk_; c += 2) {
      chunk(c, xA, xB, yA, yB);
      chunk(c + 1, yA, yB, xA, xB);
    }
    if (c < nchunk_) chunk(c, xA, xB, yA, yB);
  }

  // ---- epilogue: C fragment column (head) r, rows 4g + i of row block mb
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int tb = tbase + 16 * mb + g * 4;
    const bool vec = a.vec_out && tb + 3 < a.T;
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int l = l0 + j;
      if (l >= a.n_lv || r >= a.H) continue;
      const float bias[3] = {a.bi[l * a.H + r], a.bf[l * a.H + r], a.br[l * a.H + r]};
      T* outs[3] = {(T*)a.oi, (T*)a.of, (T*)a.orr};
      const int64_t base = (int64_t)b * a.sob + (int64_t)l * a.sol + (int64_t)r * a.soh;
      float v[3][4];
#pragma unroll
      for (int x = 0; x < 3; ++x)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[x][i] = acc[mb][j][x][i] + bias[x];
      if (a.activate) {
        float mval[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mval[i] = 1.f;
          if (HAS_MASK) {
            const int to = min(tb + i, a.T - 1);
            mval[i] = Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)to * a.smt + (int64_t)l * a.sml);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float m = (tb + i >= (1 << l) && mval[i] > 0.f) ? 1.f : 0.f;
          // compiler-emitted bf16 rounding (hardware conversion, its hazards handled)
          const float si = round_bf16_cc(dh_sigmoid(round_bf16_cc(v[0][i])));
          const float sf = round_bf16_cc(dh_sigmoid(round_bf16_cc(v[1][i])));
          const float sr = round_bf16_cc(dh_sigmoid(round_bf16_cc(v[2][i])));
          v[0][i] = si * m;
          v[1][i] = sf * m + (1.f - m);
          v[2][i] = sr;
        }
      }
#pragma unroll
      for (int x = 0; x < 3; ++x) {
        if (vec) {
          MathBf16::store4(outs[x] + base + tb, v[x]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (tb + i < a.T) outs[x][base + (int64_t)(tb + i) * a.sot] = MathBf16::out(v[x][i]);
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
  int64_t smb, smt, sml;
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
      if (ok && a.mask)
        ok = Elem<T>::load((const T*)a.mask + (int64_t)b * a.smb + (int64_t)t * a.smt + (int64_t)l * a.sml) > 0.f;
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

template <typename M, int LG, int KU>
void launch_fwd(const FwdArgs& a, dim3 grid, hipStream_t s) {
  if (a.mask)
    gate_preacts_fwd_kernel<M, LG, KU, true><<<grid, dim3(kThreads), 0, s>>>(a);
  else
    gate_preacts_fwd_kernel<M, LG, KU, false><<<grid, dim3(kThreads), 0, s>>>(a);
}

template <int LG, int MB>
void launch_fwd_lds(const FwdArgs& a, hipStream_t s) {
  constexpr int P = 64 * MB;
  dim3 grid((a.T + P - 1) / P, (a.n_lv + LG - 1) / LG, a.b);
  if (a.mask)
    gate_preacts_fwd_lds_kernel<LG, MB, true><<<grid, dim3(kThreads), 0, s>>>(a);
  else
    gate_preacts_fwd_lds_kernel<LG, MB, false><<<grid, dim3(kThreads), 0, s>>>(a);
}

// Tile per workgroup (measured on MI355X at the released widths): two levels x 64 positions once
// the launch has >= 1024 workgroups (b = 8, T = 4096: 135 us, against 143 / 155 / 224 for three /
// four / six levels -- fewer waves per SIMD -- and 169 for 2 x 128), else one level x 64 positions,
// the most workgroups for short prefills. Handing each XCD whole batch rows (a tile's level groups
// and its lagged B rows then share one L2) measured the same, 136 us, and so did rounding the hidden
// tile once instead of at the eager path's two points (the launch is not bound by that VALU work).
void dispatch_fwd_lds(const FwdArgs& a, hipStream_t s) {
  const int64_t wgs21 = (int64_t)((a.T + 63) / 64) * ((a.n_lv + 1) / 2) * a.b;
  if (wgs21 >= 1024) launch_fwd_lds<2, 1>(a, s);
  else launch_fwd_lds<1, 1>(a, s);
}

template <typename M>
void dispatch_fwd(const FwdArgs& a, int LG, int KU, dim3 grid, hipStream_t s) {
  if (LG == 1 && KU == 4) launch_fwd<M, 1, 4>(a, grid, s);
  else if (LG == 1) launch_fwd<M, 1, 1>(a, grid, s);
  else if (LG == 2 && KU == 2) launch_fwd<M, 2, 2>(a, grid, s);
  else if (LG == 2) launch_fwd<M, 2, 1>(a, grid, s);
  else if (LG == 3) launch_fwd<M, 3, 1>(a, grid, s);
  else launch_fwd<M, 4, 1>(a, grid, s);
}

extern "C" int dh_gate_preacts_fwd(int dtype, const void* A, const void* B, int64_t stride_ab, int64_t stride_at,
                                   const void* Wi, const void* Wf, const void* Wr, int64_t stride_wl,
                                   int64_t stride_wh, const float* bi, const float* bf, const float* br,
                                   const void* mask, int64_t stride_mb, int64_t stride_mt, int64_t stride_ml,
                                   void* out_i, void* out_f, void* out_r, int64_t stride_ob, int64_t stride_ot,
                                   int64_t stride_ol, int64_t stride_oh, int activate, int b, int T, int GH,
                                   int H, int n_lv, void* stream) {
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
  DH_REQUIRE(stride_ob >= 0 && stride_ot >= 0 && stride_ol >= 0 && stride_oh >= 0, DH_ERR_INVALID_ARG,
             "%s: negative output stride", who);
  const int64_t esz_in = dtype == DH_BF16 ? 2 : 4;
  DH_REQUIRE((int64_t)T * stride_at * esz_in < ((int64_t)1 << 31) &&
                 (int64_t)n_lv * stride_wl * esz_in < ((int64_t)1 << 31),
             DH_ERR_UNSUPPORTED_SHAPE, "%s: one batch row of A/B or the weights exceed 2 GiB", who);
  const size_t esz = dtype == DH_BF16 ? 2 : 4;
  const bool vec_out = stride_ot == 1 && stride_ob % 4 == 0 && stride_ol % 4 == 0 && stride_oh % 4 == 0 &&
                       aligned(out_i, 4 * esz) && aligned(out_f, 4 * esz) && aligned(out_r, 4 * esz);
  FwdArgs a{A, B, stride_ab, stride_at, Wi, Wf, Wr, stride_wl, stride_wh, bi, bf, br, mask, stride_mb, stride_mt,
            stride_ml, out_i, out_f, out_r, stride_ob, stride_ot, stride_ol, stride_oh, b, T, GH, H, n_lv,
            vec_out ? 1 : 0, activate ? 1 : 0};
  // level groups: enough workgroups to fill 256 CUs several times over, A reused across <= 4 levels
  const int tiles = (T + kTileT - 1) / kTileT;
  const int64_t tile_wgs = (int64_t)tiles * b;
  const int want_groups = (int)((1024 + tile_wgs - 1) / tile_wgs);
  int LG = (n_lv + want_groups - 1) / want_groups;
  LG = LG < 1 ? 1 : (LG > 4 ? 4 : LG);
  const int ngroups = (n_lv + LG - 1) / LG;
  const int kc = dtype == DH_BF16 ? 32 : 16;
  int KU = LG == 1 ? 4 : (LG == 2 ? 2 : 1);
  while (KU > 1 && GH % (2 * kc * KU) != 0) KU /= 2;       // GH % 64 == 0 covers 2*kc*1
  if (KU == 2 && LG == 1) KU = 1;                            // no <1, 2> instantiation
  dim3 grid(tiles, ngroups, b);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_BF16 && H <= 16)
    dispatch_fwd_lds(a, s);
  else if (dtype == DH_BF16)
    dispatch_fwd<MathBf16>(a, LG, KU, grid, s);
  else
    dispatch_fwd<MathF32>(a, LG, KU, grid, s);
  return dh_check_launch(who);
}

extern "C" int dh_gate_preacts_bwd(int dtype, const void* A, const void* B, int64_t stride_ab, int64_t stride_at,
                                   const void* Wi, const void* Wf, const void* Wr, int64_t stride_wl,
                                   int64_t stride_wh, const void* dPi, const void* dPf, const void* dPr,
                                   const void* mask, int64_t stride_mb, int64_t stride_mt, int64_t stride_ml,
                                   float* dA, float* dB,
                                   float* dWi, float* dWf, float* dWr, float* dbi, float* dbf, float* dbr, int b,
                                   int T, int GH, int H, int n_lv, void* stream) {
  const char* who = "dh_gate_preacts_bwd";
  int st = check_shapes(who, dtype, b, T, GH, H, n_lv);
  if (st) return st;
  DH_REQUIRE(A && B && Wi && Wf && Wr && dPi && dPf && dPr && dA && dB && dWi && dWf && dWr && dbi && dbf && dbr,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  hipStream_t s = (hipStream_t)stream;
  BwdArgs a{A, B, stride_ab, stride_at, Wi, Wf, Wr, stride_wl, stride_wh, dPi, dPf, dPr, mask, stride_mb,
            stride_mt, stride_ml, dA, dB, dWi, dWf, dWr, dbi, dbf, dbr, b, T, GH, H, n_lv};
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
