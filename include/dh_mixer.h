/*
 * dh_mixer.h — C-ABI of libdh_mixer.so, the gfx950 (MI355X) kernels of Dispatcher-Hybrid's gated
 * dyadic shift-and-sum mixer.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are caller-owned DEVICE pointers; the library never allocates device
 *     memory, never synchronises and never reads device memory on the host. Work is enqueued on
 *     `stream` (a hipStream_t), so every call is safe inside hipGraph stream capture.
 *   - `dtype` selects the element type of the activation/weight tensors: DH_F32 or DH_BF16.
 *     Accumulation is always fp32.
 *   - Return value: DH_OK, or a DH_ERR_* code; dh_last_error() then holds a thread-local message.
 *   - Shape limits checked by every entry point: GH % 64 == 0, 1 <= H <= 64, hd in {16,32,64,128},
 *     1 <= L <= 16, T >= 1.
 *
 * Mixer semantics (one layer, model dtype tau), for level l with lag 2^l:
 *   M[b,t,l]      = [t >= 2^l] * mask[b,t,l]                (mask optional: doc-reset mask)
 *   hid[b,t,l,:]  = relu(A[b,t,:] + M[b,t,l] * B[b,t-2^l,:])^2
 *   pre_x[b,t,l,h]= hid[b,t,l,:] . W_x[l,h,:] + b_x[l,h]      x in {i (admit), f (forget), r (transmit)}
 *   a = sigmoid(pre_i)*M ; f = sigmoid(pre_f)*M + (1-M) ; r = sigmoid(pre_r)
 *   for l < n_lv:  V[t] <- f[t,l]*V[t] + a[t,l]*r[t-2^l,l]*V[t-2^l]     (V starts at V0 = W_in.x)
 */
#ifndef DH_MIXER_H
#define DH_MIXER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DH_ABI_VERSION 19

enum dh_status {
  DH_OK = 0,
  DH_ERR_INVALID_ARG = 1,
  DH_ERR_UNSUPPORTED_SHAPE = 2,
  DH_ERR_UNSUPPORTED_DTYPE = 3,
  DH_ERR_LAUNCH_FAILED = 4,
  DH_ERR_UNIMPLEMENTED = 5
};

enum dh_dtype { DH_F32 = 0, DH_BF16 = 1 };

/* ABI version of the loaded library (DH_ABI_VERSION at build time). */
int dh_abi_version(void);

/* Thread-local message describing the last non-zero status returned on this thread. */
const char* dh_last_error(void);

/*
 * Parallel gate pre-activations (prefill / training forward).
 * Replaces the Triton kernel `_gate_pipeline_fwd` and its op `dispatcher::gate_preacts_fwd`
 * (reference dispatcher_hybrid/fused_gates.py:38-93 kernel, :186-214 op, :307-314 wrapper).
 *   A, B      (b, T, GH) rows `stride_at` elements apart, batches `stride_ab` apart; innermost dim
 *             contiguous.
 *   Wi,Wf,Wr  (>= n_lv, H, GH): level stride `stride_wl`, head stride `stride_wh` (elements);
 *             innermost contiguous.
 *   bi,bf,br  fp32, (>= n_lv, H) contiguous.
 *   mask      nullable; dtype `dtype`, value > 0 means "edge allowed", element [b,t,l] at
 *             b*stride_mb + t*stride_mt + l*stride_ml. The wrap mask t >= 2^l is always applied
 *             in-kernel.
 *   out_i/f/r dtype `dtype`, element [b,t,l,h] at b*stride_ob + t*stride_ot + l*stride_ol +
 *             h*stride_oh: (T*n_lv*H, n_lv*H, H, 1) is the reference op's contiguous (b, T, n_lv, H)
 *             layout; (H*n_lv*T, 1, T, n_lv*T) is the head-major (b, H, n_lv, T) layout that
 *             dh_level_scan_fwd reads with unit-stride loads.
 *   activate  0: write the pre-activations (the reference op's output). 1: write the level scan's
 *             gates instead: a = sigmoid(pre_i)*M, f = sigmoid(pre_f)*M + 1 - M, r = sigmoid(pre_r)
 *             with M = [t >= 2^l] * [mask > 0] (bf16: pre-activation and sigmoid rounded, as the
 *             eager path rounds them); dh_level_scan_fwd then runs with `activated`.
 */
int dh_gate_preacts_fwd(int dtype, const void* A, const void* B, int64_t stride_ab, int64_t stride_at,
                        const void* Wi, const void* Wf, const void* Wr, int64_t stride_wl,
                        int64_t stride_wh, const float* bi, const float* bf, const float* br,
                        const void* mask, int64_t stride_mb, int64_t stride_mt, int64_t stride_ml,
                        void* out_i, void* out_f, void* out_r, int64_t stride_ob, int64_t stride_ot,
                        int64_t stride_ol, int64_t stride_oh, int activate, int b, int T, int GH, int H,
                        int n_lv, void* stream);

/*
 * The mixer's input projections as one MFMA GEMM over the concatenated weights:
 *   out[s][m*ldo[s] + n] = sum_k X[m*ldx + k] * W[s][n*K + k]      s < nseg <= 3, n < N[s], m < M
 * Replaces the three nn.Linear calls V0 = linear_in(x), A = gate_hidden(x), B = gate_hidden_src(x)
 * of the parallel forward (reference dispatcher_hybrid/modeling_dispatcher.py:63-74) with one
 * launch. W[s] (N[s], K) row-major (nn.Linear weight layout), N[s] a multiple of 4; K a multiple
 * of 64 (bf16) / 32 (fp32); fp32 accumulation, one rounding per bf16 output. W, N, out, ldo are
 * host arrays of nseg entries.
 */
int dh_proj_gemm(int dtype, const void* X, int64_t ldx, int M, int K, int nseg, const void* const* W,
                 const int* N, void* const* out, const int64_t* ldo, void* stream);

/*
 * Backward of dh_gate_preacts_fwd (autograd of the fused op).
 * Replaces the Triton kernel `_gate_pipeline_bwd` and op `dispatcher::gate_preacts_bwd`
 * (reference dispatcher_hybrid/fused_gates.py:96-173 kernel, :225-257 op).
 *   dPi/dPf/dPr (b, T, n_lv, H) contiguous, dtype `dtype`; mask as in dh_gate_preacts_fwd.
 *   dA, dB      fp32 (b, T, GH) contiguous; dWi/dWf/dWr fp32 (n_lv, H, GH); dbi/dbf/dbr fp32 (n_lv, H).
 *   Every output is overwritten (the library zero-fills with a kernel, then accumulates dB, dW and
 *   db with fp32 atomics, so summation order is not deterministic, as in the reference).
 */
int dh_gate_preacts_bwd(int dtype, const void* A, const void* B, int64_t stride_ab, int64_t stride_at,
                        const void* Wi, const void* Wf, const void* Wr, int64_t stride_wl,
                        int64_t stride_wh, const void* dPi, const void* dPf, const void* dPr,
                        const void* mask, int64_t stride_mb, int64_t stride_mt, int64_t stride_ml,
                        float* dA, float* dB, float* dWi, float* dWf, float* dWr, float* dbi,
                        float* dbf, float* dbr,
                        int b, int T, int GH, int H, int n_lv, void* stream);

/*
 * Parallel level scan with the gate activations fused in (sigmoid, masks, heads-first layout).
 * Replaces reference dispatcher_hybrid/modeling_dispatcher.py:86-88, 111-121 (heads_first, the
 * admit/forget/transmit activations and the n_lv-level roll/update loop).
 *   pre_i/f/r dtype `dtype` (output of dh_gate_preacts_fwd), element [b,t,l,h] at b*stride_pb +
 *             t*stride_pt + l*stride_pl + h*stride_ph; any layout works, the head-major one
 *             (stride_pt == 1) gives unit-stride loads.
 *   mask      nullable, as in dh_gate_preacts_fwd; ignored when `activated`.
 *   activated 0: pre_i/f/r are pre-activations (sigmoid and masks applied here); 1: they are the
 *             activated, masked gates a, f, r that dh_gate_preacts_fwd writes with `activate`.
 *   V0        (b, T, H*hd): V0[b,t,h*hd+e] at b*stride_vb + t*stride_vt + h*hd + e (linear_in output).
 *   V         (b, T, H*hd) contiguous output, the scanned state in the layout linear_out consumes.
 *   ring      nullable: the decoder prefill's ring buffer V_ring (b, S, H*hd), S = 2^(ring_L+1)-2,
 *             ring_L >= n_lv (the layer's level count). For every level j < ring_L the state
 *             entering level j (V0 for j = 0; the final state for j > n_lv) of the last 2^(j+1)
 *             positions is stored at slot 2^(j+1)-2 + (t & (2^(j+1)-1)), as the reference's
 *             eager prefill stores it (dispatcher_hybrid/decoding.py:143-185); other slots are
 *             left untouched.
 */
int dh_level_scan_fwd(int dtype, const void* pre_i, const void* pre_f, const void* pre_r,
                      int64_t stride_pb, int64_t stride_pt, int64_t stride_pl, int64_t stride_ph,
                      const void* mask, int64_t stride_mb, int64_t stride_mt, int64_t stride_ml,
                      const void* V0, int64_t stride_vb, int64_t stride_vt, void* V, int b, int T, int H,
                      int hd, int n_lv, int activated, void* ring, int ring_L, void* stream);

/*
 * The feed-forward block's SwiGLU activation over n elements:
 *   out[i] = silu(gate[i]) * up[i],  silu(x) = x / (1 + e^-x)
 * Replaces F.silu(linear_gate(h)) * linear_up(h) of reference
 * dispatcher_hybrid/modeling_dispatcher.py:197 (SwiGLU.forward), two launches and a rounded
 * intermediate, at the eager rounding points: in bf16, silu is rounded to bf16 before the product
 * and the product is rounded again. dtype DH_F32 or DH_BF16; gate, up and out contiguous and
 * 16-byte aligned (out may alias gate or up). n == 0 is a no-op.
 */
int dh_silu_mul(int dtype, const void* gate, const void* up, void* out, int64_t n, void* stream);

/*
 * The feed-forward block's gate and up projections and its SwiGLU activation as one MFMA GEMM:
 *   out[m*ldo + f] = round(round(silu(round(sum_k X[m*ldx + k] Wg[f*K + k])))
 *                          * round(sum_k X[m*ldx + k] Wu[f*K + k]))            f < N, m < M
 * Replaces silu(linear_gate(h)) * linear_up(h) of reference
 * dispatcher_hybrid/modeling_dispatcher.py:188-197 (SwiGLU.forward): the two GEMMs, their bf16
 * outputs in memory and the activation pass, with the eager rounding points (each GEMM output
 * rounded to bf16, silu rounded, the product rounded) and dh_silu_mul's arithmetic. bf16 only;
 * Wg, Wu (N, K) row-major (nn.Linear weight layout); K a multiple of 64, N of 8; X, Wg, Wu and out
 * 16-byte aligned with row strides ldx >= K and ldo >= N multiples of 8 elements.
 */
int dh_proj_gemm_swiglu(int dtype, const void* X, int64_t ldx, int M, int K, const void* Wg, const void* Wu,
                        int N, void* out, int64_t ldo, void* stream);

/*
 * The parallel forward's tree mask with document resets, (b, T, L) contiguous, values 0 or 1:
 *   out[(b*T + t)*L + l] = [t >= 2^l] * [no EOT among ids[b*ids_stride + t - 2^l .. t - 1]]
 * Replaces the torch computation of the level mask times "source and destination in the same
 * document" (reference dispatcher_hybrid/modeling_dispatcher.py:282-297, 311-323: doc(t) counts the
 * EOTs before t; the edge t <- t - 2^l is kept iff doc(t) == doc(t - 2^l)). ids int64 (b, T) with row
 * stride ids_stride >= T; dtype DH_F32 or DH_BF16 (the mask's dtype); T <= 16384, L <= 30, b <= 65535;
 * out 16-byte aligned.
 */
int dh_tree_mask(int dtype, const int64_t* ids, int64_t ids_stride, int b, int T, int L, int64_t eot, void* out,
                 void* stream);

/*
 * Residual add + RMSNorm over `rows` rows of d elements (row-contiguous, 16-byte aligned):
 *   x_out = x + y;  h_out = x_out * rsqrt(mean(x_out^2) + eps) * weight
 * Replaces the add and the next nn.RMSNorm of the residual stream of reference
 * dispatcher_hybrid/modeling_dispatcher.py:210-212, :225-227 (x = x + sublayer(...); norm(x)) and
 * :341-348 (the last block's add, then norm_out). bf16: the sum is rounded to bf16 (as the eager
 * add), the norm computed in fp32 and rounded once. x_out may alias x or y. d a multiple of 8 (bf16)
 * / 4 (fp32), at most 8192 / 4096. rows == 0 is a no-op.
 */
int dh_add_rmsnorm(int dtype, const void* x, const void* y, const void* weight, float eps, void* x_out,
                   void* h_out, int64_t rows, int d, void* stream);

/*
 * One decode step of one tree layer: all L levels' gate readouts plus the L-level recurrence over
 * the ring buffers, as ONE kernel launch.
 * Computes what the Triton kernels `step_gates_kernel` + `step_scan_kernel` (reference
 * dispatcher_hybrid/fused_step.py:26-59 and :62-88) compute as launched by
 * FusedGraphedHybridDecoder._tree_step_g (reference dispatcher_hybrid/decoding.py:477-486).
 * FusedGraphedHybridDecoder runs it at batch > 1; the tests check it against the oracle and the
 * other forms (dh_decode_gates + dh_decode_scan / dh_decode_scan_out, the one-launch batch-1 step)
 * against it.
 *   A         (B, GH) destination features W1x.h1 of the current token.
 *   B_hist    (B, Tmax, GH); row t (the current token) already written.
 *   Wi,Wf,Wr  (L, H, GH) contiguous; bi,bf,br (L, H) contiguous, dtype `dtype`.
 *   t_dev     device int64[1]: the current position t (read on the device: graph-stable).
 *   rg_hist   (B, Tmax, L, H): row t is written, rows t-2^l are read.
 *   V_ring    (B, S, H*hd), S = 2^(L+1)-2: ring j occupies slots [2^(j+1)-2, 2^(j+2)-2) and holds the
 *             state entering level j; position p lives in slot 2^(j+1)-2 + (p & (2^(j+1)-1)).
 *   V0        (B, H*hd) linear_in output of the current token (ring 0's new entry).
 *   Y         (B, H*hd) output: state after level L-1.
 *   If t_dev holds a position outside [0, Tmax) the kernel writes nothing.
 *   Needs no scratch memory: one workgroup per (head, block of rows), none waiting on another.
 */
int dh_decode_mixer_step(int dtype, const void* A, const void* B_hist, const void* Wi,
                         const void* Wf, const void* Wr, const void* bi, const void* bf,
                         const void* br, const int64_t* t_dev, void* rg_hist, void* V_ring,
                         const void* V0, void* Y, int B, int Tmax, int S, int GH, int H, int hd,
                         int L, void* stream);

/*
 * Matrix-vector products of the decode step with their neighbouring elementwise work fused in.
 * Replaces the torch GEMV chain around the mixer step in FusedGraphedHybridDecoder._tree_step_g and
 * _step_all (reference dispatcher_hybrid/decoding.py:473-476, :487-488, :442) and the SwiGLU and
 * RMSNorm they call (reference dispatcher_hybrid/modeling_dispatcher.py:196-197, 207-212, 276):
 *   h = norm_w ? RMSNorm(x[b], eps) * norm_w : x[b]           (x[b] = x + x_rows[b]*x_bstride when
 *                                                              x_rows is given, else x + b*x_bstride)
 *   segment s (s < nseg <= 3): W[s] is (N[s], K) row-major; for n < N[s]:
 *     out[s][b*out_bstride[s] + t*out_t_stride[s] + n] =
 *         round(W[s][n].h)                                     plain
 *       | round(round(W[0][n].h) + resid[b, n])               resid != NULL (nseg == 1); resid[b] as x
 *       | round(round(silu(round(W[0][n].h))) * round(W[1][n].h)) into out[0]   swiglu (nseg == 2)
 *   t = *t_dev (device position; e.g. the B_hist row of the source projection), read only when
 *   some out_t_stride is non-zero. t_advance (nullable): the launch adds one to *t_advance (the
 *   decode step's position advance folded into its last launch); not allowed together with a
 *   non-zero out_t_stride. argmax_cand (nullable; B = 1, one plain segment): each workgroup also
 *   writes the best (rounded output value, row) of its rows in torch.argmax's order (NaN above all,
 *   lowest row on ties) -- dh_decode_gemv_candidates(dtype, N, K) records -- for dh_argmax_reduce:
 *   the greedy pick fused into the vocabulary head (reference modeling_dispatcher.py:426-441).
 * All activations and weights in dtype; fp32 accumulation. The array arguments W, out, out_bstride,
 * out_t_stride and N are host arrays of nseg entries. K must be a multiple of 8 (bf16) or 4 (fp32):
 * rows are read in 16-byte chunks.
 * flags: DH_GEMV_SWIGLU (the swiglu form above); DH_GEMV_FRAG_OUT: a SwiGLU launch writes out[0] in
 * 16-row MFMA fragment order instead of rows -- element (b, n) at ((n/32)*64 + ((n/8)%4)*16 + b)*8
 * + n%8, a (16, N) buffer whatever B is (N a multiple of 32, out_t_stride[0] = 0); DH_GEMV_FRAG_IN:
 * x is read in that order (x_bstride ignored). Both only on the batched matrix-core path (bf16,
 * 2 <= B <= 16, rows in place, K a multiple of 32, no argmax_cand); a launch outside it with either
 * flag is rejected. The decoder's feed-forward uses them for its hidden row h (up: FRAG_OUT, down:
 * FRAG_IN), which nothing else reads: each wave then requests its activation fragments as one
 * contiguous 1 KB per k-step (batch-16 down projection 7.6 -> 6.4 us per launch).
 */
#define DH_GEMV_SWIGLU 1
#define DH_GEMV_FRAG_OUT 2
#define DH_GEMV_FRAG_IN 4
int dh_decode_gemv(int dtype, const void* x, int64_t x_bstride, const int64_t* x_rows,
                   const void* norm_w, float eps, int nseg, const void* const* W, void* const* out,
                   const int64_t* out_bstride, const int64_t* out_t_stride, const int* N,
                   const void* resid, int64_t resid_bstride, const int64_t* resid_rows, int flags,
                   const int64_t* t_dev, int64_t* t_advance, void* argmax_cand, int B, int K,
                   void* stream);

/*
 * Number of argmax candidate records (8 bytes each: float value, int index) a batch-1
 * dh_decode_gemv launch with N output rows of K elements writes when given argmax_cand (one per
 * workgroup); 0 for unsupported arguments.
 */
int64_t dh_decode_gemv_candidates(int dtype, int N, int K);

/*
 * Banded causal attention of a whole sequence (the parallel forward and the decoder prefill of an
 * attention layer) as ONE launch: RoPE of q and k, scores over s <= t with t - s < window (window
 * 0: all s <= t), softmax, value average. Replaces the torch attention of WindowAttention.forward
 * and of the decoders' attention prefill (reference dispatcher_hybrid/modeling_dispatcher.py:
 * 168-182, dispatcher_hybrid/decoding.py:143-185).
 *   q, k, v        (B, T, H*hd) projections before RoPE, rows stride_t and batches stride_b
 *                  elements apart (the same strides for all three), 16-byte aligned rows.
 *   rope_cos/sin   (>= T, hd/2) tables.
 *   y              (B, T, H*hd) output, rows y_stride_t / batches y_stride_b apart.
 *   K_cache, V_cache  (B, H, Tmax, hd) buffers, T <= Tmax: rows [0, T) receive rope(k) and v
 *                  (bit-identical to the eager prefill's), which the attention then reads -- the
 *                  decoder caches, or scratch; strides cache_stride_b / cache_stride_h elements.
 * Two launches (the rope/copy pre-pass, then the attention).
 * bf16 only; hd in {32, 64, 128}. Rounding: each RoPE product and sum, the probabilities, the
 * output (scores stay fp32); the softmax is normalised at the end (online over 64-key blocks), so
 * outputs match the eager path to bf16 rounding.
 */
int dh_window_attention_fwd(int dtype, const void* q, const void* k, const void* v, int64_t stride_b,
                            int64_t stride_t, const void* rope_cos, const void* rope_sin, void* y,
                            int64_t y_stride_b, int64_t y_stride_t, void* K_cache, void* V_cache,
                            int64_t cache_stride_b, int64_t cache_stride_h, int Tmax, int B, int T, int H,
                            int hd, int window, void* stream);

/*
 * One decode step of a windowed RoPE attention layer: rotation of the new query and key at the
 * device position t, the cache write of (k', v) at t, the scores over the window [lo, t]
 * (lo = max(0, t+1-window), window 0 = the whole prefix), softmax and the value average, as ONE
 * launch. Replaces the torch ops of FusedGraphedHybridDecoder._attn_step_g (reference
 * dispatcher_hybrid/decoding.py:411-435) and matches the eager step (decoding.py:247-266).
 *   q, k, v          (B, H*hd) projections at t, rows qkv_bstride elements apart.
 *   rope_cos/sin     (>= Tmax, hd/2) tables in `dtype`.
 *   K_cache/V_cache  (B, H, Tmax, hd) head-major caches, updated in place at t.
 *   y                (B, H*hd) output rows y_bstride apart.
 * bf16 rounds at the eager step's points (rope products and sums, scores, scaled scores, softmax
 * output, value average); t = *t_dev outside [0, Tmax) writes nothing. hd in {16,32,64,128};
 * the attention span min(window, Tmax) (Tmax when window is 0) at most 16384.
 */
int dh_decode_attention(int dtype, const void* q, const void* k, const void* v, int64_t qkv_bstride,
                        const void* rope_cos, const void* rope_sin, void* K_cache, void* V_cache,
                        const int64_t* t_dev, void* y, int64_t y_bstride, int B, int H, int hd, int Tmax,
                        int window, void* stream);

/*
 * dh_decode_attention for small batches, as two launches over a split window: the window is cut
 * into min(16, span) segments, one workgroup per (segment, head, row) computes the segment's
 * rounded scores, maximum m_s, exp-sum l_s and unnormalised value sum o_s into `workspace`
 * (dh_decode_attention_workspace_bytes(B, H, hd) bytes), and a second launch writes
 * y = round(sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s). Same arguments, cache update and scores
 * as dh_decode_attention; the probabilities enter the value sum in fp32 (dh_decode_attention
 * rounds them to the model dtype first, as the eager bf16 step does).
 */
int64_t dh_decode_attention_workspace_bytes(int B, int H, int hd);
int dh_decode_attention_split(int dtype, const void* q, const void* k, const void* v, int64_t qkv_bstride,
                              const void* rope_cos, const void* rope_sin, void* K_cache, void* V_cache,
                              const int64_t* t_dev, void* y, int64_t y_bstride, int B, int H, int hd, int Tmax,
                              int window, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * dh_decode_mixer_step as two launches with a wider first one. The graphed decoder runs
 * dh_decode_gates with dh_decode_scan_out (below) at batch 1 and dh_decode_mixer_step at batch > 1;
 * dh_decode_scan is on no product path: it is the plain two-launch form the tests compare the
 * fused forms with.
 * dh_decode_gates runs one wave per (level, head, group of rows) -- the gate weights stream through
 * H*L compute units -- writes rg_hist[:, t] and a staging record per (b, h, l):
 *   stage[((b*H + h)*L + l)*(4 + hd) + ...] = {ig, fg, r_src, 0, V_src[0..hd)}   (fp32)
 * with ig/fg the admit/forget gates of level l at t and r_src, V_src the level-l transmit gate and
 * ring value of position t - 2^l (zeros before the sequence start). dh_decode_scan then runs the
 * L-level recurrence from the staging buffer (one workgroup per (head, row)), writing the ring
 * slots of position t and Y. Same arguments and arithmetic as dh_decode_mixer_step; `stage` holds
 * B*H*L*(4 + hd) floats of caller-provided device memory. Replaces the same Triton pair as
 * dh_decode_mixer_step (reference dispatcher_hybrid/fused_step.py:26-88, decoding.py:477-486).
 */
int dh_decode_gates(int dtype, const void* A, const void* B_hist, const void* Wi, const void* Wf,
                    const void* Wr, const void* bi, const void* bf, const void* br, const int64_t* t_dev,
                    void* rg_hist, const void* V_ring, float* stage, int B, int Tmax, int S, int GH, int H,
                    int hd, int L, void* stream);
int dh_decode_scan(int dtype, const void* V0, const float* stage, const int64_t* t_dev, void* V_ring, void* Y,
                   int B, int Tmax, int S, int H, int hd, int L, void* stream);

/*
 * Batch 1: dh_decode_scan fused into the out-projection + residual that consumes its Y (replaces,
 * with dh_decode_gates, the step kernels and the linear_out + residual of _tree_step_g, reference
 * dispatcher_hybrid/fused_step.py:62-88 and decoding.py:473-476):
 *   Y = the L-level recurrence of dh_decode_scan (ring slots of t written, Y written)
 *   out[n] = round(round(W[n] . Y) + resid[rrow*resid_stride + n])   n < N, rrow = resid_rows ? *resid_rows : 0
 * W (N, H*hd) row-major; out may alias the residual row. Every workgroup of the GEMV runs the
 * recurrence from the staging buffer; one writes the state. H*hd <= 1024; t = *t_dev outside
 * [0, Tmax) writes nothing.
 */
int dh_decode_scan_out(int dtype, const void* V0, const float* stage, const int64_t* t_dev, void* V_ring, void* Y,
                       const void* W, const void* resid, const int64_t* resid_rows, int64_t resid_stride, void* out,
                       int Tmax, int S, int H, int hd, int L, int N, void* stream);

/*
 * Greedy next token: out[b] = argmax over row b of logits (B rows of V, rows row_stride elements
 * apart), as torch.argmax: first index of the maximum, NaN above every number. Replaces the
 * torch argmax of fast_generate's greedy branch (reference dispatcher_hybrid/modeling_dispatcher.py
 * :426-441) with two short launches whose output can be fed back as the decoder's next tokens.
 * workspace: device memory of at least dh_argmax_workspace_bytes(B, V) bytes (per-slice
 * candidates); its contents on entry do not matter.
 */
int64_t dh_argmax_workspace_bytes(int B, int V);
int dh_argmax(int dtype, const void* logits, int64_t row_stride, int B, int V, int64_t* out, void* workspace,
              int64_t workspace_bytes, void* stream);

/*
 * dh_argmax without a workspace argument and without any allocation: the same two launches and
 * result as dh_argmax, the per-slice candidates held in a fixed array of device memory that the
 * library's code object carries (64 KiB per GPU, kept until the process ends). No counterpart in
 * the reference: it is for callers that cannot allocate device memory (HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). Limit: B * ceil(V / 2048) <= 8192 candidates (e.g.
 * B <= 327 rows of a 50257-token vocabulary); larger inputs return DH_ERR_UNSUPPORTED_SHAPE.
 * Every call on one GPU shares the array: calls that overlap on one GPU (other streams, other host
 * threads) race; calls ordered on one stream do not. The first call on a device looks the array's
 * address up (hipGetSymbolAddress) with that device current.
 */
int dh_argmax_noalloc(int dtype, const void* logits, int64_t row_stride, int B, int V, int64_t* out, void* stream);

/*
 * The greedy token of each of B rows from the per-workgroup candidates of a dh_decode_gemv launch
 * (argmax_cand, ncand records per row, e.g. dh_decode_gemv_candidates): out[b] = the index of the
 * best candidate in torch.argmax's order. hist (nullable): the token is also stored at
 * hist[b * hist_stride + *t_dev] when 0 <= *t_dev < hist_len (the decoder's generated-token
 * history, indexed by the position the step advanced to). ncand <= 8192.
 */
int dh_argmax_reduce(const void* cand, int B, int ncand, int64_t* out, const int64_t* t_dev, int64_t* hist,
                     int64_t hist_stride, int64_t hist_len, void* stream);

/*
 * Temperature / top-k sampling of the next token, on the device. Replaces the do_sample branch of
 * fast_generate (reference dispatcher_hybrid/modeling_dispatcher.py:426-441):
 *   l = float(logits[b]) / temperature;  l_i = -inf where l_i < kth (kth = the top_k-th largest l;
 *   every element equal to kth stays; top_k 0 = no top-k);  out[b] ~ Categorical(softmax(l)).
 * The uniform draw of row b comes from Philox4x32-10 keyed by `seed` with counter
 * (*offset_dev, b) (offset_dev nullable: counter 0), so a captured graph that advances the offset
 * draws afresh on every replay; the stream of draws is not torch's. One workgroup per row;
 * V <= 65536, 0 <= top_k <= V, temperature > 0; logits must be finite or -inf (a row with no
 * finite logit yields token 0).
 */
int dh_sample_topk(int dtype, const void* logits, int64_t row_stride, int B, int V, float temperature, int top_k,
                   uint64_t seed, const int64_t* offset_dev, int64_t* out, void* stream);
/*
 * dh_sample_topk that also writes each row's token into a position-indexed history,
 * hist[b * hist_stride + p] with p = *offset_dev when 0 <= p < hist_len (nothing otherwise): the
 * token-history update after the pick in fast_generate's sampling loop (the decoder's tok_hist),
 * folded into the sampler's launch. hist nullable (then exactly dh_sample_topk); a history needs
 * offset_dev.
 */
int dh_sample_topk_hist(int dtype, const void* logits, int64_t row_stride, int B, int V, float temperature,
                        int top_k, uint64_t seed, const int64_t* offset_dev, int64_t* out, int64_t* hist,
                        int64_t hist_stride, int64_t hist_len, void* stream);

/*
 * The two halves of dh_decode_mixer_step as separate launches, with the reference's own buffer
 * contract, for callers that drive the Triton kernels by name.
 * dh_step_gates replaces `step_gates_kernel` (reference dispatcher_hybrid/fused_step.py:26-59):
 *   IG, FG fp32 (B, L*H) outputs; rg_hist row t written.
 * dh_step_scan replaces `step_scan_kernel` (reference dispatcher_hybrid/fused_step.py:62-88).
 */
int dh_step_gates(int dtype, const void* A, const void* B_hist, const void* Wi, const void* Wf,
                  const void* Wr, const void* bi, const void* bf, const void* br,
                  const int64_t* t_dev, float* IG, float* FG, void* rg_hist, int B, int Tmax,
                  int GH, int H, int L, void* stream);

int dh_step_scan(int dtype, const void* V0, const float* IG, const float* FG, const void* rg_hist,
                 void* V_ring, const int64_t* t_dev, void* Y, int B, int Tmax, int S, int H, int hd,
                 int L, void* stream);

/*
 * One batch-1 bf16 greedy decode step of the whole model as ONE launch (one workgroup
 * per compute unit, resident for the step): the chain FusedGraphedHybridDecoder.step_greedy
 * replays as a graph of dependent launches (reference dispatcher_hybrid/decoding.py:437-488 and
 * modeling_dispatcher.py:426-441: tree steps, attention steps, final norm, vocabulary head,
 * argmax), with the same arithmetic, so the logits and the picked token equal the graphed step's.
 * Workgroups hand vectors to each other through tagged words in `scratch` (no fences, no
 * counters); every wait is bounded, and a step that times out sets the status words
 * (dh_decode_persistent_status) and writes no token.
 *   layer_table (device): n_layers records of DH_PERSISTENT_LAYER_WORDS int64 words, by field:
 *     [0] kind (0 tree layer, 1 attention layer), [1] RMSNorm1 weight,
 *     tree: [2] linear_in [3] gate_hidden [4] gate_hidden_src [5..7] gate_out, forget_out,
 *           reset_out (L, H, GH) [8..10] their biases (L, H) [11] linear_out [12] B_hist (Tmax, GH)
 *           [13] rg_hist (Tmax, L, H) [14] V_ring (2^(L+1)-2, d),
 *     attention: [2..5] linear_q, _k, _v, _out [6, 7] K, V caches (H, Tmax, 64) [8, 9] RoPE cos,
 *           sin (Tmax, 32) [10] window (0: none; its span <= DH_PERSISTENT_MAX_WINDOW),
 *     both: [15] RMSNorm2 weight [16..18] linear_gate, linear_up, linear_down.
 *   kinds (host): the n_layers kinds again, for the phase count.
 *   emb (V, d): embedding and (tied) vocabulary head; norm_out (d). *t_dev: position (advanced by
 *   one); *token: this step's token in, the greedy pick out, also stored at tok_hist[t + 1] when
 *   below hist_len (tok_hist nullable); logits (V) bf16 out.
 *   scratch: dh_decode_persistent_scratch_bytes(d, GH, H, L, ff, CUs) bytes, 256-byte aligned,
 *   zero-filled once before the first step and then kept (it holds the launch counter); steps on
 *   one scratch must not overlap. d = H*hd in {256, 512, 768, 1024}, GH <= 1024, ff <= 3072,
 *   L <= 12, head width 64 with attention layers. No counterpart in the reference (its step is a
 *   graph of launches).
 */
#define DH_PERSISTENT_LAYER_WORDS 24
#define DH_PERSISTENT_MAX_WINDOW 4096
int64_t dh_decode_persistent_scratch_bytes(int d, int GH, int H, int L, int ff, int grid);
int dh_decode_persistent_step(const int64_t* layer_table, const int* kinds, int n_layers, const void* emb,
                              const void* norm_out, float eps, int d, int GH, int H, int hd, int L, int ff, int V,
                              int Tmax, int64_t* t_dev, int64_t* token, int64_t* tok_hist, int64_t hist_len,
                              void* logits, void* scratch, int64_t scratch_bytes, void* stream);
/*
 * dh_decode_persistent_step with a timing record, for profiling the step's phases: trace
 * (caller-zeroed device memory, >= CUs x phases x 3 uint64 words) receives, per workgroup and
 * phase, the 100 MHz real-time counter at the phase's start, at the end of its wait for other
 * workgroups' words (0 where the workgroup has none) and at its end. Same arguments and results
 * otherwise; no counterpart in the reference.
 */
int dh_decode_persistent_trace(const int64_t* layer_table, const int* kinds, int n_layers, const void* emb,
                               const void* norm_out, float eps, int d, int GH, int H, int hd, int L, int ff, int V,
                               int Tmax, int64_t* t_dev, int64_t* token, int64_t* tok_hist, int64_t hist_len,
                               void* logits, void* scratch, int64_t scratch_bytes, uint64_t* trace,
                               int64_t trace_words, void* stream);
/* phases of one step for these layer kinds (0 tree, 1 attention): 5 per tree layer, 6 per
 * attention layer, 2 for the vocabulary head and the pick */
int dh_decode_persistent_phases(const int* kinds, int n_layers);
/* status words of the last persistent steps on `scratch`: out2[0] non-zero after a timeout,
 * out2[1] the first failing phase + 1 (synchronises the stream) */
int dh_decode_persistent_status(const void* scratch, uint32_t* out2, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DH_MIXER_H */
