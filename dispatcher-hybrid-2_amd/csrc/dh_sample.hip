// Next-token selection on the device, for gfx950: greedy argmax over each row of logits.
//
// Semantics follow torch.argmax as fast_generate's greedy branch calls it (reference
// dispatcher_hybrid/modeling_dispatcher.py:426-441): the index of the largest value, the first
// such index on ties, and NaN counts as larger than every number (the first NaN wins).
//
// Work decomposition: two launches. The first splits every row into slices of kSlice elements, one
// workgroup (4 wave64s) per (slice, row): each thread requests all of its elements before
// comparing any, keeps its best (value, index), and DPP wave reductions plus one LDS step give the
// slice's candidate. The second launch reduces each row's candidates with the same ordering. A
// row of a 50k vocabulary thus streams through ~25 compute units instead of one.
#include "dh_common.h"

namespace {


// a beats b: larger value, NaN above all numbers, lower index on ties
__device__ __forceinline__ bool beats(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ void dpp_pair(float& v, int& i) {
  // lanes outside ROWMASK keep their own pair (old = own value), so the comparison is a no-op there
  const float ov = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
  const int oi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROWMASK, 0xf, false);
  if (beats(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}

constexpr int kSlice = 2048;              // elements per first-pass workgroup
constexpr int kT1 = 256;                  // first-pass threads: kSlice / kT1 = 8 elements each

struct Cand {
  float v;
  int i;
};

// best (value, index) of a wave, in lane 63
__device__ __forceinline__ void wave_best(float& best, int& bidx) {
  dpp_pair<0xb1, 0xf>(best, bidx);      // quad_perm(1,0,3,2)
  dpp_pair<0x4e, 0xf>(best, bidx);      // quad_perm(2,3,0,1)
  dpp_pair<0x141, 0xf>(best, bidx);     // row_half_mirror
  dpp_pair<0x140, 0xf>(best, bidx);     // row_mirror
  dpp_pair<0x142, 0xa>(best, bidx);     // row_bcast:15 into rows 1, 3
  dpp_pair<0x143, 0xc>(best, bidx);     // row_bcast:31 into rows 2, 3
}

template <typename T>
__global__ __launch_bounds__(kT1) void argmax_slices(const T* logits, int64_t row_stride, int V, Cand* cand) {
  __shared__ Cand wb[kT1 / 64];
  const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* row = logits + (int64_t)b * row_stride;
  constexpr int PT = kSlice / kT1;
  const int base = s * kSlice;
  float x[PT];
#pragma unroll
  for (int k = 0; k < PT; ++k) x[k] = Elem<T>::load(row + min(base + tid + k * kT1, V - 1));   // clamped
  float best = x[0];
  int bidx = min(base + tid, V - 1);
#pragma unroll
  for (int k = 1; k < PT; ++k) {
    const int i = base + tid + k * kT1;
    if (i < V && beats(x[k], i, best, bidx)) {
      best = x[k];
      bidx = i;
    }
  }
  wave_best(best, bidx);
  if (lane == 63) wb[wave] = Cand{best, bidx};
  __syncthreads();
  if (tid == 0) {
    Cand c = wb[0];
#pragma unroll
    for (int w = 1; w < kT1 / 64; ++w)
      if (beats(wb[w].v, wb[w].i, c.v, c.i)) c = wb[w];
    cand[(int64_t)b * gridDim.x + s] = c;
  }
}

__global__ __launch_bounds__(64) void argmax_final(const Cand* cand, int nslice, int64_t* out) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const Cand* cb = cand + (int64_t)b * nslice;
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  for (int j = lane; j < nslice; j += 64) {
    const Cand c = cb[j];
    if (beats(c.v, c.i, best, bidx)) {
      best = c.v;
      bidx = c.i;
    }
  }
  wave_best(best, bidx);
  if (lane == 63) out[b] = bidx;
}

}  // namespace

extern "C" int64_t dh_argmax_workspace_bytes(int B, int V) {
  return (int64_t)B * ((V + kSlice - 1) / kSlice) * (int64_t)sizeof(Cand);
}

extern "C" int dh_argmax(int dtype, const void* logits, int64_t row_stride, int B, int V, int64_t* out,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  const char* who = "dh_argmax";
  DH_REQUIRE(dtype == DH_F32 || dtype == DH_BF16, DH_ERR_UNSUPPORTED_DTYPE, "%s: dtype %d", who, dtype);
  DH_REQUIRE(B >= 1 && B <= 65535 && V >= 1 && row_stride >= V, DH_ERR_INVALID_ARG, "%s: B=%d V=%d row_stride=%lld",
             who, B, V, (long long)row_stride);
  DH_REQUIRE(logits && out && workspace, DH_ERR_INVALID_ARG, "%s: null pointer argument", who);
  DH_REQUIRE(workspace_bytes >= dh_argmax_workspace_bytes(B, V), DH_ERR_INVALID_ARG,
             "%s: workspace of %lld bytes, needs %lld", who, (long long)workspace_bytes,
             (long long)dh_argmax_workspace_bytes(B, V));
  DH_REQUIRE((uintptr_t)workspace % 8 == 0, DH_ERR_INVALID_ARG, "%s: workspace needs 8-byte alignment", who);
  const int nslice = (V + kSlice - 1) / kSlice;
  Cand* cand = (Cand*)workspace;
  hipStream_t s = (hipStream_t)stream;
  dim3 g1(nslice, B);
  if (dtype == DH_BF16)
    argmax_slices<bf16_t><<<g1, kT1, 0, s>>>((const bf16_t*)logits, row_stride, V, cand);
  else
    argmax_slices<float><<<g1, kT1, 0, s>>>((const float*)logits, row_stride, V, cand);
  argmax_final<<<B, 64, 0, s>>>(cand, nslice, out);
  return dh_check_launch(who);
}
