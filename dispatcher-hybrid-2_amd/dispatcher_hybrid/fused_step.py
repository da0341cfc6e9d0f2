"""Per-token decode step of a tree layer on gfx950 HIP kernels.

Drop-in for the reference module of the same name (reference dispatcher_hybrid/fused_step.py),
whose two Triton kernels run the gate readouts over (row, level) and the level recurrence over
(row, head). FusedGraphedHybridDecoder runs them at batch 1 as ``decode_gates_scan_out``
(``dh_decode_gates``, one wave per (level, head), then the recurrence inside the out-projection
launch) and batch-1 bf16 greedy steps as ONE launch per token (``persistent_step``); at batch > 1
as ``decode_mixer_step`` (``dh_decode_mixer_step``: the layer's whole step in one launch, one
workgroup per (head, block of rows)), also the baseline the tests check the other forms against.
``decode_gates_scan`` (``dh_decode_gates`` then ``dh_decode_scan``) is the two-launch form.

Ring layout (unchanged, reference dispatcher_hybrid/decoding.py:28-37, fused_step.py:13-16):
level j's state is read only at lag 2^j, so ring j keeps 2^(j+1) slots at offset 2^(j+1)-2 and
position p lives in slot offset_j + (p & (2^(j+1)-1)).

``step_gates_kernel`` / ``step_scan_kernel`` keep the reference's launch syntax
(``kernel[grid](...)``, reference decoding.py:477-486) for callers that drive the two halves by
name; they run the two halves of the same HIP kernel as separate launches.

Importing this module loads the kernel library and raises ImportError if it is missing.
"""

import ctypes

import torch

from . import _hip


def ring_offset(j):
    return (2 << j) - 2


def ring_mask(j):
    return (2 << j) - 1


def _check_contig(name, t):
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_step(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y):
    _hip.require_gpu(A, "decode_mixer_step")
    Bb = A.shape[0]
    Tmax = B_hist.shape[1]
    L, H = Wi.shape[0], Wi.shape[1]
    d = V_ring.shape[2]
    dt = A.dtype
    for name, t in (("A", A), ("B_hist", B_hist), ("Wi", Wi), ("Wf", Wf), ("Wr", Wr), ("bi", bi),
                    ("bf", bf), ("br", br), ("rg_hist", rg_hist), ("V_ring", V_ring), ("V0", V0),
                    ("Y", Y)):
        _check_contig(name, t)
        if t.dtype != dt:
            raise TypeError(f"decode_mixer_step: {name} has dtype {t.dtype}, expected {dt}")
    if t_buf.dtype != torch.int64 or t_buf.numel() < 1:
        raise TypeError("t_buf must be an int64 device tensor")
    if tuple(rg_hist.shape) != (Bb, Tmax, L, H) or tuple(V0.shape) != (Bb, d) or tuple(Y.shape) != (Bb, d):
        raise ValueError("decode_mixer_step: inconsistent cache / buffer shapes")


def decode_mixer_step(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y):
    """One tree layer's decode step at the position held in the device tensor `t_buf`.

    A (B, GH) current destination features; B_hist (B, Tmax, GH) with row t written;
    Wi/Wf/Wr (L, H, GH); bi/bf/br (L, H); rg_hist (B, Tmax, L, H) (row t written);
    V_ring (B, S, H*hd) (slots of position t written); V0 (B, H*hd) linear_in output;
    Y (B, H*hd) output. Everything in the model dtype (fp32 or bf16), on one GPU.
    """
    _check_step(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y)
    Bb, GH = A.shape
    Tmax = B_hist.shape[1]
    L, H = Wi.shape[0], Wi.shape[1]
    S, d = V_ring.shape[1], V_ring.shape[2]
    dt = A.dtype
    p = _hip.ptr
    st = _hip.lib.dh_decode_mixer_step(
        _hip.dtype_code(dt), p(A), p(B_hist), p(Wi), p(Wf), p(Wr), p(bi), p(bf), p(br), p(t_buf),
        p(rg_hist), p(V_ring), p(V0), p(Y), Bb, Tmax, S, GH, H, d // H, L,
        _hip.stream_handle(A.device))
    _hip.check(st, "dh_decode_mixer_step")
    return Y


def decode_gemv(x, segments, t_buf, norm_weight=None, eps=None, resid=None, swiglu=False,
                x_rows=None, resid_rows=None, t_advance=None, argmax_cand=None, frag_out=False, frag_in=False):
    """Fused matrix-vector products of the decode step (``dh_decode_gemv``).

    x: (B, K) activations (or the embedding table with ``x_rows`` = token ids: row b is
    x[x_rows[b]]). segments: up to three (W, out, out_bstride, t_stride) with W (N, K) and
    out[b * out_bstride + t * t_stride + n] receiving output n of batch row b (t = t_buf[0]).
    norm_weight: RMSNorm weight applied to x first (eps defaults to the fp32 epsilon 2^-23, which
    nn.RMSNorm(eps=None) takes from torch's fp32 math type for fp32 and bf16 inputs alike). resid: (B, N) added to segment 0's result (rows through
    ``resid_rows`` when given); swiglu: segments are (gate, up) and silu(gate) * up goes to the
    gate segment's destination. t_advance: an int64 device tensor the launch adds one to (the
    decode step's position advance, folded into its last launch; outputs may then not use
    t_stride). argmax_cand: a buffer of ``gemv_candidates(dtype, N, K)`` 8-byte records (batch 1,
    one plain segment) that receives each workgroup's best (value, row) for ``argmax_reduce``.
    frag_out (a SwiGLU launch) / frag_in: the output / x in 16-row MFMA fragment order -- a (16, N)
    buffer whatever the batch, element (b, n) at ((n // 32) * 64 + (n // 8 % 4) * 16 + b) * 8 + n % 8
    -- for a hidden row only the next launch reads (bf16, 2 <= B <= 16; see the C header).
    Everything in one dtype (fp32 or bf16) on one GPU.
    """
    _hip.require_gpu(x, "decode_gemv")
    dt = x.dtype
    K = x.shape[-1]
    B = x_rows.numel() if x_rows is not None else x.shape[0]
    n = len(segments)
    Ws = (ctypes.c_void_p * n)(*[W.data_ptr() for W, _, _, _ in segments])
    outs = (ctypes.c_void_p * n)(*[o.data_ptr() for _, o, _, _ in segments])
    obs = (ctypes.c_int64 * n)(*[int(bs) for _, _, bs, _ in segments])
    ots = (ctypes.c_int64 * n)(*[int(ts) for _, _, _, ts in segments])
    Ns = (ctypes.c_int * n)(*[W.shape[0] for W, _, _, _ in segments])
    for W, o, _, _ in segments:
        if W.dtype != dt or o.dtype != dt or W.shape[1] != K or not W.is_contiguous():
            raise ValueError("decode_gemv: segment weights must be contiguous (N, K) in the activation dtype")
    if norm_weight is not None and eps is None:
        eps = torch.finfo(torch.float32).eps
    p = _hip.ptr
    st = _hip.lib.dh_decode_gemv(
        _hip.dtype_code(dt), p(x), x.stride(0), p(x_rows), p(norm_weight), float(eps or 0.0), n,
        Ws, outs, obs, ots, Ns, p(resid), resid.stride(0) if resid is not None else 0, p(resid_rows),
        int(bool(swiglu)) | (2 if frag_out else 0) | (4 if frag_in else 0), p(t_buf), p(t_advance),
        p(argmax_cand), B, K, _hip.stream_handle(x.device))
    _hip.check(st, "dh_decode_gemv")


def gemv_candidates(dtype, N, K):
    """Argmax candidate records a batch-1 decode_gemv with N rows of K elements writes."""
    return int(_hip.lib.dh_decode_gemv_candidates(_hip.dtype_code(dtype), int(N), int(K)))


def candidate_buffer(dtype, N, K, B, device):
    """A buffer for B rows of candidate records (8 bytes each), as int64 elements."""
    n = gemv_candidates(dtype, N, K)
    if n < 1:
        raise ValueError("candidate_buffer: unsupported shape")
    return torch.empty(B, n, dtype=torch.int64, device=device)


def argmax_reduce(cand, out, t_buf=None, hist=None):
    """Greedy tokens from decode_gemv's argmax candidates (``dh_argmax_reduce``): out[b] = the row
    of the best candidate of cand[b] in torch.argmax's order. hist (B, L) int64: the token is also
    stored at hist[b, t_buf[0]] when that index is inside the buffer."""
    B, ncand = cand.shape
    if cand.dtype != torch.int64 or not cand.is_contiguous():
        raise ValueError("argmax_reduce: candidates are a contiguous (B, ncand) int64 buffer")
    if out.dtype != torch.long or out.numel() != B or not out.is_contiguous():
        raise ValueError("argmax_reduce: out must be a contiguous int64 tensor of B elements")
    hs, hl = 0, 0
    if hist is not None:
        if hist.dtype != torch.long or hist.dim() != 2 or hist.shape[0] != B or hist.stride(1) != 1 or t_buf is None:
            raise ValueError("argmax_reduce: hist must be (B, L) int64 with unit inner stride, with t_buf")
        hs, hl = hist.stride(0), hist.shape[1]
    p = _hip.ptr
    st = _hip.lib.dh_argmax_reduce(p(cand), B, ncand, p(out), p(t_buf), p(hist), hs, hl,
                                   _hip.stream_handle(cand.device))
    _hip.check(st, "dh_argmax_reduce")
    return out


def stage_floats(B, H, L, hd):
    """Size (in fp32 elements) of the staging buffer decode_gates_scan needs."""
    return B * H * L * (4 + hd)


def decode_gates_scan(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y, stage):
    """decode_mixer_step as two launches (``dh_decode_gates`` then ``dh_decode_scan``): the gate
    readouts run one wave per (level, head, row group) so the gate weights stream through many
    compute units, and the recurrence reads its position-dependent sources from the fp32 staging
    buffer `stage` (``stage_floats(B, H, L, hd)`` elements) the first launch fills. Same arguments,
    state updates and arithmetic as decode_mixer_step."""
    _check_step(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y)
    Bb, Tmax, GH = B_hist.shape
    S, d = V_ring.shape[1], V_ring.shape[2]
    L, H = Wi.shape[0], Wi.shape[1]
    hd = d // H
    if stage.dtype != torch.float32 or not stage.is_contiguous() or stage.numel() < stage_floats(Bb, H, L, hd):
        raise ValueError(f"decode_gates_scan: stage must be a contiguous fp32 buffer of >= "
                         f"{stage_floats(Bb, H, L, hd)} elements")
    p = _hip.ptr
    code = _hip.dtype_code(A.dtype)
    stream = _hip.stream_handle(A.device)
    st = _hip.lib.dh_decode_gates(code, p(A), p(B_hist), p(Wi), p(Wf), p(Wr), p(bi), p(bf), p(br),
                                  p(t_buf), p(rg_hist), p(V_ring), p(stage), Bb, Tmax, S, GH, H, hd, L,
                                  stream)
    _hip.check(st, "dh_decode_gates")
    st = _hip.lib.dh_decode_scan(code, p(V0), p(stage), p(t_buf), p(V_ring), p(Y), Bb, Tmax, S, H, hd,
                                 L, stream)
    _hip.check(st, "dh_decode_scan")


def scan_out_supported(B, d):
    """dh_decode_scan_out covers batch 1 with d = H*hd <= 1024."""
    return B == 1 and d <= 1024


def decode_gates_scan_out(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y, stage,
                          W_out, resid, out, resid_rows=None):
    """decode_gates_scan followed by the layer's out-projection + residual, out = round(round(
    W_out . Y) + resid) (reference decoding.py:473-476), in two launches at batch 1:
    ``dh_decode_gates`` and ``dh_decode_scan_out``, which runs the recurrence in every workgroup of
    the out-projection GEMV (workgroup 0 writes the ring slots and Y). resid: rows of N elements
    (row resid_rows[0] when given, else row 0); out: (1, N), may be the residual row itself."""
    _check_step(A, B_hist, Wi, Wf, Wr, bi, bf, br, t_buf, rg_hist, V_ring, V0, Y)
    Bb, Tmax, GH = B_hist.shape
    S, d = V_ring.shape[1], V_ring.shape[2]
    L, H = Wi.shape[0], Wi.shape[1]
    hd = d // H
    if not scan_out_supported(Bb, d):
        raise ValueError(f"decode_gates_scan_out: batch {Bb}, d {d} (needs batch 1, d <= 1024)")
    if stage.dtype != torch.float32 or not stage.is_contiguous() or stage.numel() < stage_floats(Bb, H, L, hd):
        raise ValueError("decode_gates_scan_out: stage too small or not contiguous fp32")
    N = W_out.shape[0]
    for name, t in (("W_out", W_out), ("resid", resid), ("out", out)):
        if t.dtype != A.dtype or t.stride(-1) != 1:
            raise ValueError(f"decode_gates_scan_out: {name} must be {A.dtype} with a unit inner stride")
    if tuple(W_out.shape) != (N, d) or not W_out.is_contiguous() or resid.shape[-1] != N or out.numel() < N:
        raise ValueError("decode_gates_scan_out: W_out (N, d), resid rows of N and out of N elements expected")
    p = _hip.ptr
    code = _hip.dtype_code(A.dtype)
    stream = _hip.stream_handle(A.device)
    st = _hip.lib.dh_decode_gates(code, p(A), p(B_hist), p(Wi), p(Wf), p(Wr), p(bi), p(bf), p(br),
                                  p(t_buf), p(rg_hist), p(V_ring), p(stage), Bb, Tmax, S, GH, H, hd, L,
                                  stream)
    _hip.check(st, "dh_decode_gates")
    rstride = resid.stride(0) if resid.dim() > 1 else N
    st = _hip.lib.dh_decode_scan_out(code, p(V0), p(stage), p(t_buf), p(V_ring), p(Y), p(W_out), p(resid),
                                     p(resid_rows), rstride, p(out), Tmax, S, H, hd, L, N, stream)
    _hip.check(st, "dh_decode_scan_out")


class _Launcher:
    """`kernel[grid](*args, **meta)` call syntax of a Triton kernel, mapped onto a HIP entry."""

    def __init__(self, fn, name):
        self._fn = fn
        self.__name__ = name

    def __getitem__(self, grid):
        return lambda *args, **meta: self._fn(tuple(grid), *args, **meta)


def _step_gates(grid, A, B_hist, Wi, Wf, Wr, bi, bf, br, T_buf, IG, FG, RG_hist, T_max,
                GH=None, H=None, L=None, BK=None):
    """Reference contract (fused_step.py:26-59): grid (B, L); writes IG/FG fp32 (B, L*H) and
    RG_hist[:, t] (model dtype). BK is accepted for compatibility; the HIP kernel tiles itself."""
    _hip.require_gpu(A, "step_gates_kernel")
    Bb = A.shape[0]
    GH = A.shape[1] if GH is None else GH
    L = Wi.shape[0] if L is None else L
    H = Wi.shape[1] if H is None else H
    if grid[0] != Bb or (len(grid) > 1 and grid[1] != L):
        raise ValueError(f"step_gates_kernel grid {grid} must be (B={Bb}, L={L})")
    p = _hip.ptr
    st = _hip.lib.dh_step_gates(_hip.dtype_code(A.dtype), p(A), p(B_hist), p(Wi), p(Wf), p(Wr),
                                p(bi), p(bf), p(br), p(T_buf), p(IG), p(FG), p(RG_hist),
                                Bb, int(T_max), GH, H, L, _hip.stream_handle(A.device))
    _hip.check(st, "dh_step_gates")


def _step_scan(grid, V0, IG, FG, RG_hist, V_ring, T_buf, Y, T_max, S, L=None, HD=None, H=None):
    """Reference contract (fused_step.py:62-88): grid (B, H); writes the ring slots of position
    t for levels 0..L-1 and Y."""
    _hip.require_gpu(V0, "step_scan_kernel")
    Bb, d = V0.shape
    if H is None or HD is None or L is None:
        raise ValueError("step_scan_kernel needs L=, HD= and H=")
    if grid[0] != Bb or (len(grid) > 1 and grid[1] != H):
        raise ValueError(f"step_scan_kernel grid {grid} must be (B={Bb}, H={H})")
    p = _hip.ptr
    st = _hip.lib.dh_step_scan(_hip.dtype_code(V0.dtype), p(V0), p(IG), p(FG), p(RG_hist),
                               p(V_ring), p(T_buf), p(Y), Bb, int(T_max), int(S), H, HD, L,
                               _hip.stream_handle(V0.device))
    _hip.check(st, "dh_step_scan")


step_gates_kernel = _Launcher(_step_gates, "step_gates_kernel")
step_scan_kernel = _Launcher(_step_scan, "step_scan_kernel")


def attention_workspace(B, H, hd, device):
    """Workspace of the split-window attention step (``dh_decode_attention_split``)."""
    n = int(_hip.lib.dh_decode_attention_workspace_bytes(B, H, hd))
    return torch.empty((n + 3) // 4, dtype=torch.float32, device=device)


def decode_attention(q, k, v, rope_cos, rope_sin, K_cache, V_cache, t_buf, y, window, workspace=None):
    """One decode step of a windowed RoPE attention layer (``dh_decode_attention``).

    q, k, v: (B, H*hd) projections at the device position t = t_buf[0]; K_cache/V_cache:
    (B, H, Tmax, hd) head-major caches (row t written here); rope_cos/rope_sin: (>= Tmax, hd/2)
    tables; y: (B, H*hd) receives softmax((q' . K) / sqrt(hd)) . V over [max(0, t+1-window), t]
    (the whole prefix when window is 0). One launch; same rounding points as the eager step
    (reference dispatcher_hybrid/decoding.py:247-266, :411-435). With a `workspace`
    (attention_workspace(B, H, hd, device)) the window is split over up to 16 workgroups per head
    and combined in a second launch (``dh_decode_attention_split``), the probabilities then kept in
    fp32: the small-batch form.
    """
    _hip.require_gpu(q, "decode_attention")
    B, H, Tmax, hd = K_cache.shape
    dt = q.dtype
    for name, x in (("k", k), ("v", v), ("rope_cos", rope_cos), ("rope_sin", rope_sin),
                    ("K_cache", K_cache), ("V_cache", V_cache), ("y", y)):
        if x.dtype != dt:
            raise TypeError(f"decode_attention: {name} is {x.dtype}, expected {dt}")
    for name, x in (("q", q), ("k", k), ("v", v), ("y", y)):
        if x.shape[0] != B or x.shape[-1] != H * hd or x.stride(-1) != 1:
            raise ValueError(f"decode_attention: {name} must be ({B}, {H * hd}) with unit inner stride")
    if not (q.stride(0) == k.stride(0) == v.stride(0)):
        raise ValueError("decode_attention: q, k and v need one row stride")
    if not (K_cache.is_contiguous() and V_cache.is_contiguous() and V_cache.shape == K_cache.shape):
        raise ValueError("decode_attention: caches must be contiguous (B, H, Tmax, hd)")
    if not (rope_cos.is_contiguous() and rope_sin.is_contiguous()) or rope_cos.shape[0] < Tmax \
            or rope_cos.shape[-1] != hd // 2:
        raise ValueError("decode_attention: rope tables must be contiguous (>= Tmax, hd/2)")
    p = _hip.ptr
    if workspace is not None:
        if workspace.dtype != torch.float32 or not workspace.is_contiguous():
            raise ValueError("decode_attention: workspace must be a contiguous fp32 tensor")
        st = _hip.lib.dh_decode_attention_split(
            _hip.dtype_code(dt), p(q), p(k), p(v), q.stride(0), p(rope_cos), p(rope_sin),
            p(K_cache), p(V_cache), p(t_buf), p(y), y.stride(0), B, H, hd, Tmax, int(window),
            p(workspace), workspace.numel() * 4, _hip.stream_handle(q.device))
        _hip.check(st, "dh_decode_attention_split")
        return
    st = _hip.lib.dh_decode_attention(
        _hip.dtype_code(dt), p(q), p(k), p(v), q.stride(0), p(rope_cos), p(rope_sin),
        p(K_cache), p(V_cache), p(t_buf), p(y), y.stride(0), B, H, hd, Tmax, int(window),
        _hip.stream_handle(q.device))
    _hip.check(st, "dh_decode_attention")


def argmax_workspace(B, V, device):
    """A candidate buffer for argmax_tokens over (B, V) logits (uint8 device tensor)."""
    return torch.empty(max(int(_hip.lib.dh_argmax_workspace_bytes(B, V)), 4096), dtype=torch.uint8, device=device)


def argmax_tokens(logits, out=None, workspace=None):
    """Greedy next tokens on the device (``dh_argmax``): out[b] = logits[b].argmax() as int64,
    first index on ties, NaN above every number (torch.argmax's rule). logits: (B, V) fp32 or bf16
    with a unit inner stride; returns `out` (allocated when None).

    workspace: the candidate buffer (argmax_workspace(B, V, device)). A step captured into a HIP
    graph must pass one it owns for the graph's lifetime; without it a per-device buffer is used
    that a later call with more candidates replaces (freeing the old one), which only eager
    callers may rely on."""
    _hip.require_gpu(logits, "argmax_tokens")
    if logits.dim() != 2 or logits.stride(-1) != 1:
        raise ValueError("argmax_tokens: logits must be (B, V) with a unit inner stride")
    B, V = logits.shape
    if out is None:
        out = torch.empty(B, dtype=torch.long, device=logits.device)
    if out.dtype != torch.long or out.numel() != B or not out.is_contiguous():
        raise ValueError("argmax_tokens: out must be a contiguous int64 tensor of B elements")
    nbytes = int(_hip.lib.dh_argmax_workspace_bytes(B, V))
    ws = workspace
    if ws is not None:
        if ws.dtype != torch.uint8 or ws.device != logits.device or not ws.is_contiguous() or ws.numel() < nbytes:
            raise ValueError(f"argmax_tokens: workspace must be a contiguous uint8 tensor of >= {nbytes} bytes "
                             f"on the logits' device")
    else:
        ws = _ARGMAX_WS.get(logits.device)
        if ws is None or ws.numel() < nbytes:
            ws = argmax_workspace(B, V, logits.device)
            _ARGMAX_WS[logits.device] = ws
    st = _hip.lib.dh_argmax(_hip.dtype_code(logits.dtype), _hip.ptr(logits), logits.stride(0), B, V,
                            _hip.ptr(out), _hip.ptr(ws), ws.numel(), _hip.stream_handle(logits.device))
    _hip.check(st, "dh_argmax")
    return out


_ARGMAX_WS = {}           # per-device candidate buffer of eager argmax_tokens calls, grown on demand


def argmax_tokens_noalloc(logits, out):
    """argmax_tokens without any allocation (``dh_argmax_noalloc``), for code that cannot allocate
    device memory, such as a step under HIP graph capture: the candidates live in the library's
    fixed per-GPU scratch (B * ceil(V / 2048) <= 8192). `out`: caller-provided contiguous int64 of B
    elements. Calls that overlap on one GPU (other streams or threads) race on that scratch."""
    _hip.require_gpu(logits, "argmax_tokens_noalloc")
    if logits.dim() != 2 or logits.stride(-1) != 1:
        raise ValueError("argmax_tokens_noalloc: logits must be (B, V) with a unit inner stride")
    B, V = logits.shape
    if out.dtype != torch.long or out.numel() != B or not out.is_contiguous() or out.device != logits.device:
        raise ValueError("argmax_tokens_noalloc: out must be a contiguous int64 tensor of B elements on the logits' device")
    st = _hip.lib.dh_argmax_noalloc(_hip.dtype_code(logits.dtype), _hip.ptr(logits), logits.stride(0), B, V,
                                    _hip.ptr(out), _hip.stream_handle(logits.device))
    _hip.check(st, "dh_argmax_noalloc")
    return out


def sample_tokens(logits, temperature=1.0, top_k=None, seed=0, offset=None, out=None, hist=None):
    """Temperature / top-k sampling on the device (``dh_sample_topk``), the do_sample branch of
    fast_generate (reference modeling_dispatcher.py:426-441): logits.float() / temperature, every
    element below the top_k-th largest masked out (ties with it kept), one draw per row from
    softmax. The draw of row b comes from Philox4x32-10 keyed by `seed` with counter (offset[0], b):
    pass the decoder's device position as `offset` so each step draws afresh (also under graph
    replay). logits: (B, V) fp32 or bf16, unit inner stride, V <= 65536. Returns int64 `out`.

    hist: an optional (B, L) int64 token history (unit inner stride); the kernel also writes each
    row's token to hist[b, offset[0]] when 0 <= offset[0] < L (``dh_sample_topk_hist``), the
    history update after the pick, with no launch of its own. Needs `offset`."""
    _hip.require_gpu(logits, "sample_tokens")
    if logits.dim() != 2 or logits.stride(-1) != 1:
        raise ValueError("sample_tokens: logits must be (B, V) with a unit inner stride")
    B, V = logits.shape
    k = 0 if top_k is None else int(top_k)
    if not 0 < k <= V and top_k is not None:
        raise ValueError(f"sample_tokens: top_k={top_k} out of range for {V} logits")
    if not temperature > 0:
        raise ValueError(f"sample_tokens: temperature {temperature} must be positive")
    if offset is not None and (offset.dtype != torch.long or offset.device != logits.device):
        raise ValueError("sample_tokens: offset must be an int64 tensor on the logits' device")
    if out is None:
        out = torch.empty(B, dtype=torch.long, device=logits.device)
    if out.dtype != torch.long or out.numel() != B or not out.is_contiguous():
        raise ValueError("sample_tokens: out must be a contiguous int64 tensor of B elements")
    if hist is None:
        st = _hip.lib.dh_sample_topk(_hip.dtype_code(logits.dtype), _hip.ptr(logits), logits.stride(0), B, V,
                                     ctypes.c_float(float(temperature)), k, ctypes.c_uint64(int(seed) & (2 ** 64 - 1)),
                                     _hip.ptr(offset), _hip.ptr(out), _hip.stream_handle(logits.device))
        _hip.check(st, "dh_sample_topk")
        return out
    if offset is None:
        raise ValueError("sample_tokens: a token history needs the position (offset)")
    if (hist.dtype != torch.long or hist.dim() != 2 or hist.shape[0] != B or hist.stride(1) != 1
            or hist.device != logits.device):
        raise ValueError("sample_tokens: hist must be a (B, L) int64 tensor with a unit inner stride on the "
                         "logits' device")
    st = _hip.lib.dh_sample_topk_hist(_hip.dtype_code(logits.dtype), _hip.ptr(logits), logits.stride(0), B, V,
                                      ctypes.c_float(float(temperature)), k,
                                      ctypes.c_uint64(int(seed) & (2 ** 64 - 1)), _hip.ptr(offset), _hip.ptr(out),
                                      _hip.ptr(hist), hist.stride(0), hist.shape[1], _hip.stream_handle(logits.device))
    _hip.check(st, "dh_sample_topk_hist")
    return out


# ---------------------------------------------------------------------------------------------
# One-launch batch-1 step (dh_decode_persistent_step)
# ---------------------------------------------------------------------------------------------
LAYER_WORDS = 24          # DH_PERSISTENT_LAYER_WORDS
MAX_WINDOW = 4096         # DH_PERSISTENT_MAX_WINDOW


def persistent_fits(d, GH, H, hd, L, ff, grid):
    """Whether dh_decode_persistent_step takes these dimensions on `grid` compute units (the
    checks the entry point makes: every output row of a phase has a wave, 16 attention segments
    per head fit two per workgroup)."""
    return (d in (256, 512, 768, 1024) and H * hd == d and 64 <= GH <= 1024 and GH % 64 == 0
            and 64 <= ff <= 3072 and ff % 32 == 0 and 1 <= L <= 12 and H * L <= 768
            and grid * 4 >= d and grid * 12 >= d + 2 * GH and grid * 12 >= ff and grid * 2 >= H * 16
            and grid * 4 >= H * L
            and grid <= 256)


def persistent_scratch_bytes(d, GH, H, L, ff, grid):
    """Scratch bytes of dh_decode_persistent_step for these dimensions and `grid` compute units."""
    return int(_hip.lib.dh_decode_persistent_scratch_bytes(int(d), int(GH), int(H), int(L), int(ff), int(grid)))


def persistent_phases(kinds):
    """Phases of one one-launch step for these layer kinds."""
    n = len(kinds)
    return int(_hip.lib.dh_decode_persistent_phases((ctypes.c_int * n)(*[int(k) for k in kinds]), n))


def persistent_step(table, kinds, emb, norm_out, eps, dims, t_buf, token_buf, tok_hist, logits, scratch, trace=None):
    """One batch-1 bf16 greedy decode step of the whole model as one cooperative launch.

    table: (n_layers, LAYER_WORDS) int64 device tensor of weight / cache addresses (field order of
    include/dh_mixer.h); kinds: host list of layer kinds (0 tree, 1 attention); dims: (d, GH, H, hd,
    L, ff, V, Tmax). Reads the token in token_buf at position t_buf[0]; writes the greedy pick to
    token_buf and tok_hist[0, t + 1], the logits (1, V) and advances t_buf. scratch: zero-filled once
    (persistent_scratch_bytes), then kept with the decoder. trace (optional): a zeroed uint64-sized
    (CUs, phases, 3) int64 tensor that receives each workgroup's real-time counter at every phase's
    start, wait end and end (dh_decode_persistent_trace)."""
    n = len(kinds)
    karr = (ctypes.c_int * n)(*[int(k) for k in kinds])
    d, GH, H, hd, L, ff, V, Tmax = (int(v) for v in dims)
    p = _hip.ptr
    hist_len = tok_hist.shape[-1] if tok_hist is not None else 0
    args = (p(table), karr, n, p(emb), p(norm_out), float(eps), d, GH, H, hd, L, ff, V, Tmax, p(t_buf), p(token_buf),
            p(tok_hist), hist_len, p(logits), p(scratch), scratch.numel() * scratch.element_size())
    if trace is None:
        st = _hip.lib.dh_decode_persistent_step(*args, _hip.stream_handle(emb.device))
        _hip.check(st, "dh_decode_persistent_step")
    else:
        if trace.dtype != torch.int64 or not trace.is_contiguous():
            raise ValueError("persistent_step: trace must be a contiguous int64 tensor")
        st = _hip.lib.dh_decode_persistent_trace(*args, p(trace), trace.numel(), _hip.stream_handle(emb.device))
        _hip.check(st, "dh_decode_persistent_trace")


def persistent_status(scratch):
    """(timed out, first failing phase + 1) of the steps run on `scratch` so far (synchronises)."""
    out = (ctypes.c_uint32 * 2)()
    _hip.check(_hip.lib.dh_decode_persistent_status(_hip.ptr(scratch), out, _hip.stream_handle(scratch.device)),
               "dh_decode_persistent_status")
    return int(out[0]), int(out[1])
