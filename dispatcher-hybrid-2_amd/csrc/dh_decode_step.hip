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
// Work decomposition (MI355X: 256 CUs in 8 XCDs, wave64):
//   grid = H * L workgroups of 256 threads. Workgroup (h, l) streams its three GH-long weight rows
//   W_x[l, h, :] once and reduces them against every batch row's hidden vector, so gate weights
//   are read once per step whatever the batch size. The workgroup that completes a head's last
//   level (a device-scope counter per head) runs that head's L-level recurrence for all rows: one
//   lane per element of the head's hd-wide slice, all L ring/rg sources prefetched up front since
//   the slot written at t never aliases the slot read at t - 2^l. When H is a multiple of 8, the
//   L workgroups of one head share blockIdx % 8, i.e. one XCD under round-robin dispatch, so the
//   hand-off stays within one L2.
#include "dh_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxL = 16;
constexpr int kRowChunk = 8;         // batch rows reduced together per weight pass
constexpr int kCounterStride = 32;   // uint32s between per-head counters (128-byte lines)

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
  unsigned int* counters;
  int B, Tmax, S, GH, H, hd, L;
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

template <typename T>
__global__ __launch_bounds__(kThreads) void decode_mixer_step_kernel(StepArgs a) {
  const int64_t t = *a.t_dev;
  if (t < 0 || t >= a.Tmax) return;  // every workgroup leaves: no counter is touched
  int h, l;
  block_coords(blockIdx.x, a.H, a.L, h, l);
  gates_phase<T>(a, h, l, t);

  // publish this workgroup's IG/FG/rg stores device-wide, then count the level in
  __threadfence();
  __syncthreads();
  __shared__ int is_last;
  if (threadIdx.x == 0) {
    unsigned int* c = a.counters + (int64_t)h * kCounterStride;
    const unsigned int prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == (unsigned int)(a.L - 1));
    if (is_last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();  // acquire the other levels' IG/FG
  scan_phase<T>(a, h, t);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void step_gates_kernel(StepArgs a) {
  const int64_t t = *a.t_dev;
  if (t < 0 || t >= a.Tmax) return;
  int h, l;
  block_coords(blockIdx.x, a.H, a.L, h, l);
  gates_phase<T>(a, h, l, t);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void step_scan_kernel(StepArgs a) {
  const int64_t t = *a.t_dev;
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

}  // namespace

extern "C" size_t dh_decode_workspace_bytes(int B, int L, int H) {
  if (B < 1 || L < 1 || H < 1) return 0;
  return (size_t)H * kCounterStride * sizeof(unsigned int) + 2 * (size_t)B * L * H * sizeof(float);
}

extern "C" int dh_decode_mixer_step(int dtype, const void* A, const void* B_hist, const void* Wi,
                                    const void* Wf, const void* Wr, const void* bi, const void* bf,
                                    const void* br, const int64_t* t_dev, void* rg_hist,
                                    void* V_ring, const void* V0, void* Y, void* workspace, int B,
                                    int Tmax, int S, int GH, int H, int hd, int L, void* stream) {
  const char* who = "dh_decode_mixer_step";
  int st = check_common(who, dtype, B, Tmax, GH, H, hd, L);
  if (st) return st;
  DH_REQUIRE(S == (int)ring_offset(L), DH_ERR_INVALID_ARG, "%s: S=%d but L=%d needs %lld ring slots", who, S, L,
             (long long)ring_offset(L));
  DH_REQUIRE(A && B_hist && Wi && Wf && Wr && bi && bf && br && t_dev && rg_hist && V_ring && V0 && Y && workspace,
             DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(aligned(A, 16) && aligned(B_hist, 16) && aligned(Wi, 16) && aligned(Wf, 16) && aligned(Wr, 16) &&
                 aligned(workspace, 128),
             DH_ERR_INVALID_ARG, "%s: A/B_hist/W need 16-byte and workspace 128-byte alignment", who);
  StepArgs a{A, B_hist, Wi, Wf, Wr, bi, bf, br, t_dev, rg_hist, V_ring, V0, Y, nullptr, nullptr, nullptr,
             B, Tmax, S, GH, H, hd, L};
  a.counters = (unsigned int*)workspace;
  a.IG = (float*)((char*)workspace + (size_t)H * kCounterStride * sizeof(unsigned int));
  a.FG = a.IG + (size_t)B * L * H;
  dim3 grid(H * L), block(kThreads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32)
    decode_mixer_step_kernel<float><<<grid, block, 0, s>>>(a);
  else
    decode_mixer_step_kernel<bf16_t><<<grid, block, 0, s>>>(a);
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
  StepArgs a{A, B_hist, Wi, Wf, Wr, bi, bf, br, t_dev, rg_hist, nullptr, nullptr, nullptr, IG, FG, nullptr,
             B, Tmax, 0, GH, H, 64, L};
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
             V_ring, V0, Y, (float*)IG, (float*)FG, nullptr, B, Tmax, S, 64, H, hd, L};
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DH_F32)
    step_scan_kernel<float><<<dim3(H), dim3(kThreads), 0, s>>>(a);
  else
    step_scan_kernel<bf16_t><<<dim3(H), dim3(kThreads), 0, s>>>(a);
  return dh_check_launch(who);
}
