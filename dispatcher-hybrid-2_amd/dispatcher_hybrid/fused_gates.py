"""Fused gate pipeline of the parallel (prefill / training) forward, on gfx950 HIP kernels.

    model.enable_fused_gates()

Drop-in for the reference module of the same name (reference dispatcher_hybrid/fused_gates.py):
the custom ops ``dispatcher::gate_preacts_fwd`` / ``dispatcher::gate_preacts_bwd`` keep their
schemas (reference :186-190, :225-229), fake implementations and autograd registration, and
``fused_gate_preacts`` keeps its signature (reference :307-314). They compute

    hidden = relu(A + m * roll(B, 2^l))^2            (never materialised)
    pre_x  = hidden . W_x[l] + b_x[l]                x in {i, f, r}

in one kernel (``dh_gate_preacts_fwd``). Dtype rule: bf16 (and fp16) inputs compute in bf16 with
fp32 accumulation and return bf16, like the reference; fp32 inputs compute and return fp32 (the
reference op rounds fp32 models to bf16, which cannot meet a 1e-4 relative tolerance).

Also registered here: ``dispatcher::level_scan_fwd``, the sigmoid/mask/level-scan half of the
mixer (``dh_level_scan_fwd``), which the reference runs as eager torch ops
(reference dispatcher_hybrid/modeling_dispatcher.py:86-88, 111-121).

``silu_mul`` is the feed-forward block's SwiGLU activation in one launch (``dh_silu_mul``);
``add_rmsnorm`` a residual add and the RMSNorm after it (``dh_add_rmsnorm``).

Importing this module loads the kernel library and raises ImportError if it is missing.
"""

import ctypes
import weakref
from typing import List, Optional

import torch

from . import _hip


def _compute_dtype(x):
    return torch.float32 if x.dtype == torch.float32 else torch.bfloat16


def _mask_view(mask, cd):
    """(b, T, n_lv) mask in dtype `cd` and its element strides (any layout; no copy if already cd)."""
    if mask is None:
        return None, 0, 0, 0
    m = mask.to(cd)
    return m, m.stride(0), m.stride(1), m.stride(2)


def _preacts_launch(A_, B_, Wi_, Wf_, Wr_, bi_, bf_, br_, mask, outs, ostrides, activate, n_lv, what):
    b, T, GH = A_.shape
    H = Wi_.shape[1]
    cd = A_.dtype
    m_, smb, smt, sml = _mask_view(mask, cd)
    p = _hip.ptr
    st = _hip.lib.dh_gate_preacts_fwd(
        _hip.dtype_code(cd), p(A_), p(B_), A_.stride(0), A_.stride(1),
        p(Wi_), p(Wf_), p(Wr_), Wi_.stride(0), Wi_.stride(1),
        p(bi_), p(bf_), p(br_), p(m_), smb, smt, sml,
        p(outs[0]), p(outs[1]), p(outs[2]), *ostrides, int(activate),
        b, T, GH, H, n_lv, _hip.stream_handle(A_.device))
    _hip.check(st, what)


# fp32 copies of bf16 gate biases (the kernel reads fp32 biases), one per bias tensor, refreshed
# when the tensor's version counter moves (an in-place update): three cast launches per layer and
# forward otherwise. A HIP graph captured over a forward keeps the copy it was captured with.
# (keyed by id, with a weak reference that drops the entry when the tensor goes: a tensor cannot
# be a WeakKeyDictionary key, whose lookups compare keys with ==)
_BIAS_F32 = {}


def _bias_f32(v, n_lv):
    if v.dtype == torch.float32 or (v.requires_grad and torch.is_grad_enabled()):
        return v[:n_lv].contiguous().float()
    k = id(v)
    ent = _BIAS_F32.get(k)
    if ent is None or ent[0]() is not v or ent[1] != v._version or ent[2] != n_lv:
        ref = weakref.ref(v, lambda _r, k=k: _BIAS_F32.pop(k, None))
        ent = (ref, v._version, n_lv, v[:n_lv].contiguous().float())
        _BIAS_F32[k] = ent
    return ent[3]


def _prep_gate_inputs(A, B, Wi, Wf, Wr, bi, bf, br, n_lv):
    cd = _compute_dtype(A)
    A_ = A.contiguous().to(cd)
    B_ = B.contiguous().to(cd)
    Wi_, Wf_, Wr_ = (w[:n_lv].contiguous().to(cd) for w in (Wi, Wf, Wr))
    bi_, bf_, br_ = (_bias_f32(v, n_lv) for v in (bi, bf, br))
    return A_, B_, Wi_, Wf_, Wr_, bi_, bf_, br_


# ---------------------------------------------------------------------------------------------
# dispatcher::gate_preacts_fwd
# ---------------------------------------------------------------------------------------------
@torch.library.custom_op("dispatcher::gate_preacts_fwd", mutates_args=(), device_types="cuda")
def _gate_preacts_fwd_op(A: torch.Tensor, B: torch.Tensor,
                         Wi: torch.Tensor, Wf: torch.Tensor, Wr: torch.Tensor,
                         bi: torch.Tensor, bf: torch.Tensor, br: torch.Tensor,
                         n_lv: int, mask: Optional[torch.Tensor]) -> List[torch.Tensor]:
    b, T, GH = A.shape
    H = Wi.shape[1]
    cd = _compute_dtype(A)
    outs = [torch.empty(b, T, n_lv, H, device=A.device, dtype=cd) for _ in range(3)]
    if b == 0 or T == 0:
        return outs
    ins = _prep_gate_inputs(A, B, Wi, Wf, Wr, bi, bf, br, n_lv)
    o = outs[0]
    _preacts_launch(*ins, mask, outs, (o.stride(0), o.stride(1), o.stride(2), o.stride(3)), 0, n_lv,
                    "dispatcher::gate_preacts_fwd")
    return outs


@_gate_preacts_fwd_op.register_fake
def _(A, B, Wi, Wf, Wr, bi, bf, br, n_lv, mask):
    b, T, _ = A.shape
    H = Wi.shape[1]
    cd = _compute_dtype(A)
    return [A.new_empty(b, T, n_lv, H, dtype=cd) for _ in range(3)]


# ---------------------------------------------------------------------------------------------
# dispatcher::gate_preacts_bwd
# ---------------------------------------------------------------------------------------------
@torch.library.custom_op("dispatcher::gate_preacts_bwd", mutates_args=(), device_types="cuda")
def _gate_preacts_bwd_op(A: torch.Tensor, B: torch.Tensor,
                         Wi: torch.Tensor, Wf: torch.Tensor, Wr: torch.Tensor,
                         dPi: torch.Tensor, dPf: torch.Tensor, dPr: torch.Tensor,
                         n_lv: int, mask: Optional[torch.Tensor]) -> List[torch.Tensor]:
    b, T, GH = A.shape
    H = Wi.shape[1]
    dev = A.device
    f32 = torch.float32
    outs = [torch.empty(b, T, GH, device=dev, dtype=f32), torch.empty(b, T, GH, device=dev, dtype=f32)]
    outs += [torch.empty(n_lv, H, GH, device=dev, dtype=f32) for _ in range(3)]
    outs += [torch.empty(n_lv, H, device=dev, dtype=f32) for _ in range(3)]
    if b == 0 or T == 0:
        for o in outs:
            o.zero_()
        return outs
    cd = _compute_dtype(A)
    A_ = A.contiguous().to(cd)
    B_ = B.contiguous().to(cd)
    Wi_, Wf_, Wr_ = (w[:n_lv].contiguous().to(cd) for w in (Wi, Wf, Wr))
    dPi_, dPf_, dPr_ = (g.contiguous().to(cd) for g in (dPi, dPf, dPr))
    m_, smb, smt, sml = _mask_view(mask, cd)
    p = _hip.ptr
    st = _hip.lib.dh_gate_preacts_bwd(
        _hip.dtype_code(cd), p(A_), p(B_), A_.stride(0), A_.stride(1),
        p(Wi_), p(Wf_), p(Wr_), Wi_.stride(0), Wi_.stride(1),
        p(dPi_), p(dPf_), p(dPr_), p(m_), smb, smt, sml,
        *[p(o) for o in outs], b, T, GH, H, n_lv, _hip.stream_handle(dev))
    _hip.check(st, "dispatcher::gate_preacts_bwd")
    return outs


@_gate_preacts_bwd_op.register_fake
def _(A, B, Wi, Wf, Wr, dPi, dPf, dPr, n_lv, mask):
    b, T, GH = A.shape
    H = Wi.shape[1]
    f32 = torch.float32
    return ([A.new_empty(b, T, GH, dtype=f32), A.new_empty(b, T, GH, dtype=f32)]
            + [A.new_empty(n_lv, H, GH, dtype=f32) for _ in range(3)]
            + [A.new_empty(n_lv, H, dtype=f32) for _ in range(3)])


def _setup_context(ctx, inputs, output):
    A, B, Wi, Wf, Wr, bi, bf, br, n_lv, mask = inputs
    ctx.save_for_backward(A, B, Wi, Wf, Wr)
    ctx.n_lv = n_lv
    ctx.mask = mask
    ctx.dtypes = (A.dtype, B.dtype, Wi.dtype, bi.dtype)


def _backward(ctx, grads):
    dPi, dPf, dPr = grads
    A, B, Wi, Wf, Wr = ctx.saved_tensors
    n_lv = ctx.n_lv
    z = lambda g: g if g is not None else torch.zeros(
        A.shape[0], A.shape[1], n_lv, Wi.shape[1], device=A.device, dtype=_compute_dtype(A))
    dA, dB, dWi, dWf, dWr, dbi, dbf, dbr = torch.ops.dispatcher.gate_preacts_bwd(
        A, B, Wi, Wf, Wr, z(dPi), z(dPf), z(dPr), n_lv, ctx.mask)
    a_dt, b_dt, w_dt, bias_dt = ctx.dtypes
    levels = Wi.shape[0]

    def pad(g, dt):
        if g.shape[0] == levels:
            return g.to(dt)
        out = torch.zeros((levels,) + tuple(g.shape[1:]), device=g.device, dtype=dt)
        out[:n_lv] = g
        return out

    return (dA.to(a_dt), dB.to(b_dt), pad(dWi, w_dt), pad(dWf, w_dt), pad(dWr, w_dt),
            pad(dbi, bias_dt), pad(dbf, bias_dt), pad(dbr, bias_dt), None, None)


torch.library.register_autograd("dispatcher::gate_preacts_fwd", _backward, setup_context=_setup_context)


def fused_gate_preacts(A, B, Wi, Wf, Wr, bi, bf, br, n_lv, mask=None):
    """(pre_i, pre_f, pre_r), each (b, T, n_lv, H), differentiable and opaque to torch.compile.

    Equal to einsum('btlg,lhg->btlh', relu(A.unsqueeze(2) + m * roll(B, 2^l))**2, W_x[:n_lv]) +
    b_x[:n_lv]; `mask` is the optional (b, T, n_lv) doc-reset mask, the wrap mask t >= 2^l is
    always applied. Same signature as reference dispatcher_hybrid/fused_gates.py:307-314.
    """
    out = torch.ops.dispatcher.gate_preacts_fwd(A, B, Wi, Wf, Wr, bi, bf, br, n_lv, mask)
    return out[0], out[1], out[2]


# ---------------------------------------------------------------------------------------------
# dispatcher::level_scan_fwd
# ---------------------------------------------------------------------------------------------
@torch.library.custom_op("dispatcher::level_scan_fwd", mutates_args=(), device_types="cuda")
def _level_scan_fwd_op(pre_i: torch.Tensor, pre_f: torch.Tensor, pre_r: torch.Tensor,
                       mask: Optional[torch.Tensor], V0: torch.Tensor, num_heads: int,
                       n_lv: int) -> torch.Tensor:
    b, T, d = V0.shape
    out = torch.empty(b, T, d, device=V0.device, dtype=V0.dtype)
    if b == 0 or T == 0:
        return out
    _scan_launch(pre_i, pre_f, pre_r, mask, V0, out, num_heads, n_lv, 0, "dispatcher::level_scan_fwd")
    return out


def _scan_launch(pre_i, pre_f, pre_r, mask, V0, out, num_heads, n_lv, activated, what, ring=None, ring_L=0):
    b, T, d = V0.shape
    cd = V0.dtype
    V0_ = V0 if V0.stride(-1) == 1 else V0.contiguous()
    pi, pf, pr = (g.to(cd) for g in (pre_i, pre_f, pre_r))       # keeps each tensor's layout
    if not (pi.stride() == pf.stride() == pr.stride()):
        pi, pf, pr = pi.contiguous(), pf.contiguous(), pr.contiguous()
    m_, smb, smt, sml = _mask_view(mask, cd)
    p = _hip.ptr
    st = _hip.lib.dh_level_scan_fwd(
        _hip.dtype_code(cd), p(pi), p(pf), p(pr), *pi.stride(), p(m_), smb, smt, sml,
        p(V0_), V0_.stride(0), V0_.stride(1), p(out), b, T, num_heads, d // num_heads, n_lv,
        int(activated), p(ring), int(ring_L), _hip.stream_handle(V0.device))
    _hip.check(st, what)


@_level_scan_fwd_op.register_fake
def _(pre_i, pre_f, pre_r, mask, V0, num_heads, n_lv):
    return torch.empty_like(V0)


def fused_level_scan(pre_i, pre_f, pre_r, mask, V0, num_heads, n_lv):
    """Scanned mixer state (b, T, d) from the pre-activations and V0 = linear_in(x) (b, T, d).

    Applies a = sigmoid(pre_i)*M, f = sigmoid(pre_f)*M + (1-M), r = sigmoid(pre_r) and the n_lv
    updates V[t] <- f*V[t] + a*r[t-2^l]*V[t-2^l] (reference dispatcher_hybrid/modeling_dispatcher.py
    :111-121), with M = [t >= 2^l] * mask. The result is in (b, T, H*hd) layout, ready for
    linear_out (no heads-first transposes). Inference only (no autograd).
    """
    return torch.ops.dispatcher.level_scan_fwd(pre_i, pre_f, pre_r, mask, V0, num_heads, n_lv)


# ---------------------------------------------------------------------------------------------
# dispatcher::gate_scan_fwd -- the whole inference gate path in two launches
# ---------------------------------------------------------------------------------------------
@torch.library.custom_op("dispatcher::gate_scan_fwd", mutates_args=(), device_types="cuda")
def _gate_scan_fwd_op(A: torch.Tensor, B: torch.Tensor,
                      Wi: torch.Tensor, Wf: torch.Tensor, Wr: torch.Tensor,
                      bi: torch.Tensor, bf: torch.Tensor, br: torch.Tensor,
                      mask: Optional[torch.Tensor], V0: torch.Tensor, num_heads: int,
                      n_lv: int) -> torch.Tensor:
    b, T, d = V0.shape
    out = torch.empty(b, T, d, device=V0.device, dtype=V0.dtype)
    if b == 0 or T == 0:
        return out
    ins = _prep_gate_inputs(A, B, Wi, Wf, Wr, bi, bf, br, n_lv)
    H = num_heads
    # activated gates in the head-major (b, H, n_lv, T) layout: unit stride along t for the scan
    g = torch.empty(3, b, H, n_lv, T, device=V0.device, dtype=ins[0].dtype)
    gates = [g[i].permute(0, 3, 2, 1) for i in range(3)]              # logical (b, T, n_lv, H)
    _preacts_launch(*ins, mask, gates, gates[0].stride(), 1, n_lv, "dispatcher::gate_scan_fwd")
    cd = ins[0].dtype
    res = out if V0.dtype == cd else torch.empty(b, T, d, device=V0.device, dtype=cd)
    _scan_launch(gates[0], gates[1], gates[2], None, V0.to(cd), res, H, n_lv, 1, "dispatcher::gate_scan_fwd")
    if res is not out:
        out.copy_(res)
    return out


@_gate_scan_fwd_op.register_fake
def _(A, B, Wi, Wf, Wr, bi, bf, br, mask, V0, num_heads, n_lv):
    return torch.empty_like(V0)


def fused_gate_scan(A, B, Wi, Wf, Wr, bi, bf, br, n_lv, mask, V0, num_heads):
    """Scanned mixer state (b, T, d) straight from the gate hiddens A = gate_hidden(x),
    B = gate_hidden_src(x) and V0 = linear_in(x): the pre-activations are computed, activated and
    masked in one kernel (written head-major, never in the reference op's layout) and the level
    scan consumes them in a second. Inference only (no autograd); equal to
    fused_level_scan(*fused_gate_preacts(...), mask, V0, num_heads, n_lv) up to the bf16 rounding
    of the activated gates, which follows the eager path (reference
    dispatcher_hybrid/modeling_dispatcher.py:86-88, 100-121)."""
    return torch.ops.dispatcher.gate_scan_fwd(A, B, Wi, Wf, Wr, bi, bf, br, mask, V0, num_heads, n_lv)


def prefill_gate_scan(A, B, Wi, Wf, Wr, bi, bf, br, V0, num_heads, rg_hist, V_ring):
    """Decoder prefill of one tree layer through the parallel kernels: the scanned state (b, T, d)
    plus the decode state the eager prefill fills (reference dispatcher_hybrid/decoding.py:143-185)
    -- rg_hist[:, :T] for every one of the layer's L levels (beyond the prompt's horizon the wrap
    mask is zero, so the transmit gate is sigmoid(relu(A)^2 . W_r + b_r), the eager prefill's
    formula) and, in V_ring, the state entering each level of the last 2^(j+1) positions. Two
    launches: dh_gate_preacts_fwd (activated, all L levels, head-major) and dh_level_scan_fwd over
    the active levels with the ring output; one strided copy moves the transmit gates into
    rg_hist. A, B, V0: (b, T, .) in the state's dtype; no doc-reset mask (a decoder prompt is one
    document)."""
    b, T, d = V0.shape
    L = Wi.shape[0]
    H = num_heads
    cd = _compute_dtype(A)
    if rg_hist.dtype != cd or V_ring.dtype != cd or rg_hist.shape[2] != L:
        raise ValueError("prefill_gate_scan: rg_hist / V_ring must be (b, Tmax, L, H) / (b, S, d) in the compute dtype")
    ins = _prep_gate_inputs(A, B, Wi, Wf, Wr, bi, bf, br, L)
    g = torch.empty(3, b, H, L, T, device=V0.device, dtype=cd)
    gates = [g[i].permute(0, 3, 2, 1) for i in range(3)]              # logical (b, T, L, H)
    _preacts_launch(*ins, None, gates, gates[0].stride(), 1, L, "prefill_gate_scan")
    rg_hist[:, :T].copy_(gates[2])
    n_lv = min(L, T.bit_length())                                       # levels with a source
    out = torch.empty(b, T, d, device=V0.device, dtype=cd)
    _scan_launch(gates[0], gates[1], gates[2], None, V0.to(cd), out, H, n_lv, 1, "prefill_gate_scan",
                 ring=V_ring, ring_L=L)
    return out


def fused_projections(x, weights):
    """[x . W_s^T for W_s in weights] as ONE MFMA GEMM launch (``dh_proj_gemm``) over the
    concatenated weights: the mixer's V0 = linear_in(x), A = gate_hidden(x), B = gate_hidden_src(x)
    (reference dispatcher_hybrid/modeling_dispatcher.py:63-74). x: (..., K) in fp32 or bf16,
    weights: up to three (N_s, K) tensors of x's dtype. Inference only (no autograd)."""
    _hip.require_gpu(x, "fused_projections")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    n = len(weights)
    for w in weights:
        if w.dtype != x.dtype or w.dim() != 2 or w.shape[1] != K or not w.is_contiguous():
            raise ValueError("fused_projections: weights must be contiguous (N, K) tensors of x's dtype")
    outs = [torch.empty(*x.shape[:-1], w.shape[0], device=x.device, dtype=x.dtype) for w in weights]
    if M == 0:
        return outs
    Ws = (ctypes.c_void_p * n)(*[w.data_ptr() for w in weights])
    Ns = (ctypes.c_int * n)(*[w.shape[0] for w in weights])
    Os = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    Ls = (ctypes.c_int64 * n)(*[w.shape[0] for w in weights])
    st = _hip.lib.dh_proj_gemm(_hip.dtype_code(x.dtype), _hip.ptr(x2), x2.stride(0), M, K, n, Ws, Ns, Os, Ls,
                               _hip.stream_handle(x.device))
    _hip.check(st, "dh_proj_gemm")
    return outs


def projections_fit(x, linears):
    """True when dh_proj_gemm takes x . W^T for these bias-free nn.Linear layers: CUDA input, weights
    of x's dtype, K a multiple of 64 (bf16) / 32 (fp32), output widths multiples of 4."""
    return (x.is_cuda and len(linears) <= 3 and all(l.bias is None for l in linears)
            and all(l.weight.dtype == x.dtype and l.weight.is_contiguous() for l in linears)
            and x.shape[-1] % (64 if x.dtype == torch.bfloat16 else 32) == 0
            and all(l.weight.shape[0] % 4 == 0 for l in linears))


# Rows above which the three library GEMMs (hipBLASLt through nn.Linear) beat dh_proj_gemm for the
# mixer's input projections (measured on MI355X at K = 1024, N = 3 x 1024, bf16, HIP events over 20
# launches: dh_proj_gemm 36 / 61 / 92 / 96 / 190 us against 58 / 63 / 79 / 90 / 173 us for the
# library at M = 4096 / 8192 / 12288 / 16384 / 32768; below 4096 rows dh_proj_gemm takes half the
# library's time or less).
PROJ_GEMM_MAX_ROWS = 8192


def input_projections(x, mixer):
    """V0 = linear_in(x), A = gate_hidden(x), B = gate_hidden_src(x) (reference
    modeling_dispatcher.py:63-74): one dh_proj_gemm launch for a bias-free mixer whose widths the
    kernel takes (K a multiple of 64 for bf16 / 32 for fp32, widths multiples of 4) up to
    PROJ_GEMM_MAX_ROWS rows (the C2 forward and the decoders' prompt prefills); the three nn.Linear
    calls for more rows (the C5 forward's 32768), where the library is faster, and for other layers.
    Inference only."""
    lins = (mixer.linear_in, mixer.gate_hidden, mixer.gate_hidden_src)
    rows = x.numel() // max(x.shape[-1], 1)
    if rows <= PROJ_GEMM_MAX_ROWS and projections_fit(x, lins):
        return fused_projections(x, [l.weight for l in lins])
    return tuple(l(x) for l in lins)


# Rows up to which one dh_proj_gemm launch beats the library, measured on MI355X in captured graphs
# (bf16; us, ours against the library): an attention layer's q, k, v (three 1024-wide nn.Linear
# GEMMs, K = 1024) 13.3 / 23.8 at 1024 rows, 19.6 / 29.7 at 2048, 30.0 / 37.4 at 4096, 60 / 59 at
# 8192; over 18 distinct weights per graph, as in the forward, a single 1024 x 1024 output
# projection (the mixer's and attention's linear_out) 6.7 / 8.9 at 1024, 9.1 / 10.4 at 2048,
# 12.9 / 13.0 at 4096, and the SwiGLU down projection (1024 x 2816) 12.1 / 14.0 at 1024, 19.8 / 18.8
# at 2048 (the launches of at most 512 tiles keep two or three K tiles in flight).
QKV_GEMM_MAX_ROWS = 4096
OUT_GEMM_MAX_ROWS = 2048
DOWN_GEMM_MAX_ROWS = 1024


def project(x, linears, max_rows):
    """[l(x) for l in linears] (bias-free nn.Linear layers over the same input) as one dh_proj_gemm
    launch when x has at most max_rows rows and the kernel takes the shapes (projections_fit), else
    the library calls. Inference only."""
    rows = x.numel() // max(x.shape[-1], 1)
    if rows <= max_rows and projections_fit(x, linears):
        return fused_projections(x, [l.weight for l in linears])
    return [l(x) for l in linears]


def swiglu_fits(x, gate, up):
    """True when dh_proj_gemm_swiglu takes silu(gate(x)) * up(x) for these bias-free nn.Linear
    layers: a bf16 CUDA input with 16-byte aligned rows, bf16 contiguous weights of one shape, K a
    multiple of 64 and N of 8."""
    K = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and gate.bias is None and up.bias is None
            and gate.weight.dtype == up.weight.dtype == torch.bfloat16
            and gate.weight.shape == up.weight.shape and gate.weight.shape[1] == K
            and gate.weight.is_contiguous() and up.weight.is_contiguous()
            and K % 64 == 0 and gate.weight.shape[0] % 8 == 0)


def fused_swiglu(x, w_gate, w_up):
    """silu(x . w_gate^T) * (x . w_up^T) as ONE launch (``dh_proj_gemm_swiglu``): the SwiGLU block's
    gate and up GEMMs and its activation (reference dispatcher_hybrid/modeling_dispatcher.py:188-197)
    at the eager rounding points -- both GEMM outputs rounded to bf16, silu rounded, the product
    rounded -- without the two GEMM outputs ever reaching memory. x: (..., K) bf16; w_gate, w_up:
    (N, K) bf16. Returns (..., N). Inference only (no autograd)."""
    _hip.require_gpu(x, "fused_swiglu")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.clone(memory_format=torch.contiguous_format)      # a fresh, aligned copy
    N = w_gate.shape[0]
    if (x.dtype != torch.bfloat16 or w_gate.dtype != torch.bfloat16 or w_up.dtype != torch.bfloat16
            or w_gate.shape != (N, K) or w_up.shape != (N, K) or not w_gate.is_contiguous()
            or not w_up.is_contiguous()):
        raise ValueError("fused_swiglu: bf16 x (..., K) and contiguous bf16 (N, K) gate and up weights")
    out = torch.empty(*x.shape[:-1], N, device=x.device, dtype=x.dtype)
    M = x2.shape[0]
    if M == 0:
        return out
    st = _hip.lib.dh_proj_gemm_swiglu(_hip.DH_BF16, _hip.ptr(x2), x2.stride(0), M, K, _hip.ptr(w_gate),
                                      _hip.ptr(w_up), N, _hip.ptr(out), N, _hip.stream_handle(x.device))
    _hip.check(st, "dh_proj_gemm_swiglu")
    return out


TREE_MASK_MAX_LEN = 16384
TREE_MASK_MAX_ROWS = 65535
TREE_MASK_MAX_LEVELS = 30


def tree_mask(input_ids, levels, eot, dtype):
    """The parallel forward's tree mask with document resets in ONE launch (``dh_tree_mask``):
    mask[b, t, l] = 1 iff t >= 2^l and no EOT lies among input_ids[b, t-2^l .. t-1], else 0 (the
    level mask times "source and destination in the same document", reference
    dispatcher_hybrid/modeling_dispatcher.py:282-297, 311-323). input_ids: (b, T) int64 CUDA tensor;
    dtype float32 or bfloat16. Returns a contiguous (b, T, levels) tensor of exact 0s and 1s."""
    _hip.require_gpu(input_ids, "tree_mask")
    if input_ids.dim() != 2 or input_ids.dtype != torch.int64 or dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("tree_mask: (b, T) int64 input_ids and a float32 or bfloat16 mask dtype")
    b, T = input_ids.shape
    if not (1 <= levels <= TREE_MASK_MAX_LEVELS) or T > TREE_MASK_MAX_LEN or b > TREE_MASK_MAX_ROWS:
        raise ValueError(f"tree_mask: levels={levels} (1..{TREE_MASK_MAX_LEVELS}), T={T} (<= {TREE_MASK_MAX_LEN}), "
                         f"b={b} (<= {TREE_MASK_MAX_ROWS})")
    # rows of unit stride at least T apart (an expanded batch, stride 0, is copied)
    ids = input_ids if input_ids.stride(1) == 1 and input_ids.stride(0) >= T else input_ids.contiguous()
    out = torch.empty(b, T, levels, device=ids.device, dtype=dtype)
    if b == 0 or T == 0:
        return out
    st = _hip.lib.dh_tree_mask(_hip.dtype_code(dtype), _hip.ptr(ids), ids.stride(0), b, T, levels, int(eot),
                               _hip.ptr(out), _hip.stream_handle(ids.device))
    _hip.check(st, "dh_tree_mask")
    return out


def silu_mul(gate, up, out=None):
    """silu(gate) * up in one launch (``dh_silu_mul``): the SwiGLU activation of reference
    dispatcher_hybrid/modeling_dispatcher.py:197, F.silu(linear_gate(h)) * linear_up(h), at its
    eager rounding points (bf16: silu rounded to bf16, then the product rounded). gate and up:
    same shape, fp32 or bf16 CUDA tensors; out (optional) may be gate or up. Inference only."""
    _hip.require_gpu(gate, "silu_mul")
    if up.shape != gate.shape or up.dtype != gate.dtype or gate.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("silu_mul: gate and up need one shape and one dtype, fp32 or bf16")
    # contiguous and 16-byte aligned (a view at an odd storage offset is copied)
    g = gate.contiguous() if gate.is_contiguous() and gate.data_ptr() % 16 == 0 else gate.clone()
    u = up.contiguous() if up.is_contiguous() and up.data_ptr() % 16 == 0 else up.clone()
    o = torch.empty_like(g) if out is None else out
    if o.shape != g.shape or o.dtype != g.dtype or not o.is_contiguous():
        raise ValueError("silu_mul: out must be a contiguous tensor of gate's shape and dtype")
    st = _hip.lib.dh_silu_mul(_hip.dtype_code(g.dtype), _hip.ptr(g), _hip.ptr(u), _hip.ptr(o), g.numel(),
                              _hip.stream_handle(g.device))
    _hip.check(st, "dh_silu_mul")
    return o


def _rms_eps(norm):
    # nn.RMSNorm(eps=None) uses the machine epsilon of its fp32 computation type
    return norm.eps if norm.eps is not None else torch.finfo(torch.float32).eps


def add_rmsnorm_fits(d, dtype):
    """Whether dh_add_rmsnorm takes rows of width d in `dtype`: fp32 or bf16, d a multiple of the
    16-byte chunk (8 bf16 or 4 fp32 elements) and at most 64 lanes x 16 chunks of it (8192 bf16,
    4096 fp32 elements)."""
    if dtype not in (torch.float32, torch.bfloat16):
        return False
    v = 8 if dtype == torch.bfloat16 else 4
    return v <= d <= 1024 * v and d % v == 0


def add_rmsnorm(x, y, norm, out=None):
    """(x + y, norm(x + y)) in one launch (``dh_add_rmsnorm``): the residual add of a block and the
    RMSNorm after it (reference dispatcher_hybrid/modeling_dispatcher.py:210-212, 225-227, 341-348).
    x, y: (..., d) fp32 or bf16 CUDA tensors of one shape and dtype; norm: an nn.RMSNorm over d with
    a weight of x's dtype. The sum is written to `out` (x itself may be passed) or a new tensor.
    Inference only."""
    _hip.require_gpu(x, "add_rmsnorm")
    d = x.shape[-1]
    w = norm.weight
    if (y.shape != x.shape or y.dtype != x.dtype or x.dtype not in (torch.float32, torch.bfloat16)
            or w is None or w.dtype != x.dtype or tuple(w.shape) != (d,) or tuple(norm.normalized_shape) != (d,)):
        raise ValueError("add_rmsnorm: x, y need one shape and dtype (fp32 or bf16) and a weighted RMSNorm over "
                         "their last dimension in that dtype")
    xs = x if x.is_contiguous() and x.data_ptr() % 16 == 0 else x.contiguous().clone()
    ys = y if y.is_contiguous() and y.data_ptr() % 16 == 0 else y.contiguous().clone()
    xo = torch.empty_like(xs) if out is None else out
    if xo.shape != x.shape or xo.dtype != x.dtype or not xo.is_contiguous():
        raise ValueError("add_rmsnorm: out must be a contiguous tensor of x's shape and dtype")
    h = torch.empty_like(xs)
    st = _hip.lib.dh_add_rmsnorm(_hip.dtype_code(x.dtype), _hip.ptr(xs), _hip.ptr(ys), _hip.ptr(w),
                                 float(_rms_eps(norm)), _hip.ptr(xo), _hip.ptr(h), xs.numel() // d, d,
                                 _hip.stream_handle(x.device))
    _hip.check(st, "dh_add_rmsnorm")
    return xo, h
