"""Kernel-level parity of the HIP entry points against the float64 C oracle (oracle/dh_oracle.c).

Bars: fp32 kernels within 1e-5 relative of the oracle (the north-star fp32 bar is 1e-4); bf16
kernels against the oracle evaluated on the same bf16-rounded inputs, within bf16 rounding;
ring-buffer slot indexing bit-exact (integer-valued known-answer test with saturated gates).
"""

import numpy as np
import pytest
import torch

from helpers import rel_err
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cuda(x, dtype):
    return torch.as_tensor(np.asarray(x), dtype=torch.float64).to(dtype).to(DEV)


def _np(t):
    return t.detach().double().cpu().numpy()


# --------------------------------------------------------------------------------------------
# gate pre-activations
# --------------------------------------------------------------------------------------------
PREACT_CASES = [
    # b, T, GH, H, L, with_mask
    (1, 1, 64, 2, 3, False),
    (2, 37, 64, 4, 6, True),
    (1, 100, 128, 20, 7, True),          # H > 16: two MFMA column tiles, one partly padded
    (1, 256, 512, 8, 8, False),          # C1 shape (d 512, 8 levels, T 256)
    (2, 200, 1024, 16, 12, True),        # release widths
    # level groups: the host gives each workgroup LG levels so that tiles x groups >= 1024
    # (fp32 streaming kernel: level groups of 2, 3, 4; bf16 LDS kernel: two levels per workgroup
    # from 1024 workgroups, with a partial last tile and a one-level last group in the second)
    (3, 4096, 128, 4, 12, False),        # 192 tiles -> LG 2, two k-chunks per step
    (11, 1500, 64, 4, 12, True),         # 264 tiles -> LG 3, last group 2 levels, last tile partial
    (6, 4096, 64, 4, 12, True),          # 384 tiles -> LG 4
    (2, 4096, 128, 8, 12, True),         # bf16: 768 two-level workgroups -> one level per workgroup
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", PREACT_CASES)
def test_gate_preacts_fwd_matches_oracle(case, dtype):
    from dispatcher_hybrid import fused_gates  # noqa: F401
    b, T, GH, H, L, with_mask = case
    print(f"gate_preacts case={case} dtype={dtype}", flush=True)
    rng = np.random.default_rng(hash(case) % 2**32)
    n_lv = om.active_levels(L, T)
    A = rng.normal(size=(b, T, GH)) * 0.7
    B = rng.normal(size=(b, T, GH)) * 0.7
    Ws = [rng.normal(size=(L, H, GH)) / np.sqrt(GH) for _ in range(3)]
    bs = [rng.normal(size=(L, H)) for _ in range(3)]
    mask = (rng.random((b, T, L)) > 0.25).astype(np.float64) if with_mask else None
    tA, tB = _cuda(A, dtype), _cuda(B, dtype)
    tW = [_cuda(w, dtype) for w in Ws]
    tb = [_cuda(x, torch.float32) for x in bs]
    tm = None if mask is None else _cuda(mask, dtype)[..., :n_lv]
    outs = torch.ops.dispatcher.gate_preacts_fwd(tA, tB, *tW, *tb, n_lv, tm)
    torch.cuda.synchronize()
    # oracle on exactly the values the kernel saw
    ref = om.gate_preacts(_np(tA), _np(tB), *[_np(w) for w in tW], *bs, n_lv,
                          None if mask is None else mask[..., :n_lv])
    for x in range(3):
        assert outs[x].dtype == dtype and tuple(outs[x].shape) == (b, T, n_lv, H)
        err = rel_err(_np(outs[x]), ref[x])
        # bf16: a+b and hid rounded to bf16 (as the eager bf16 path rounds), output rounded
        assert err < (1e-5 if dtype == torch.float32 else 1.5e-2), f"gate {x}: rel {err:.3e}"


def test_gate_preacts_reference_dtype_rule():
    """bf16 in -> bf16 out (the reference op's rule); fp16 is computed in bf16 too."""
    b, T, GH, H, L = 1, 8, 64, 2, 3
    A = torch.randn(b, T, GH, device=DEV, dtype=torch.float16)
    W = torch.randn(L, H, GH, device=DEV)
    bias = torch.zeros(L, H, device=DEV)
    outs = torch.ops.dispatcher.gate_preacts_fwd(A, A, W, W, W, bias, bias, bias, 3, None)
    assert all(o.dtype == torch.bfloat16 for o in outs)


# --------------------------------------------------------------------------------------------
# level scan
# --------------------------------------------------------------------------------------------
SCAN_CASES = [
    # b, T, H, hd, n_lv, with_mask
    (1, 1, 2, 64, 1, False),
    (2, 45, 4, 16, 6, True),
    (1, 256, 8, 64, 8, False),           # C1
    (1, 600, 2, 32, 10, True),           # PPT = 2
    (2, 1024, 16, 64, 11, True),         # C2 length
    (1, 1500, 4, 32, 11, True),          # two positions per thread
    (1, 4096, 2, 128, 12, True),         # full context, hd 128
    (1, 5000, 2, 64, 12, False),         # past 4096 positions: the 512-thread kernel
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", SCAN_CASES)
def test_level_scan_matches_oracle(case, dtype):
    from dispatcher_hybrid.fused_gates import fused_level_scan
    b, T, H, hd, n_lv, with_mask = case
    print(f"level_scan case={case} dtype={dtype}", flush=True)
    rng = np.random.default_rng(hash(case) % 2**32)
    pres = [rng.normal(size=(b, T, n_lv, H)) * 2 for _ in range(3)]
    V0 = rng.normal(size=(b, T, H * hd))
    mask = (rng.random((b, T, n_lv)) > 0.2).astype(np.float64) if with_mask else None
    tp = [_cuda(p, dtype) for p in pres]
    tV0 = _cuda(V0, dtype)
    tm = None if mask is None else _cuda(mask, dtype)
    V = fused_level_scan(*tp, tm, tV0, H, n_lv)
    torch.cuda.synchronize()
    ref = om.level_scan(*[_np(p) for p in tp], _np(tV0), H, mask)
    err = rel_err(_np(V), ref)
    assert err < (1e-5 if dtype == torch.float32 else 2e-2), f"rel {err:.3e}"


@pytest.mark.parametrize("T,n_lv,ring_L", [(3000, 12, 12), (1500, 11, 12), (300, 9, 10)])
def test_level_scan_ring_output(T, n_lv, ring_L):
    """The decoder-prefill output of the scan (fp32, pre-activation mode with a mask): ring slab j
    holds, at slot 2^(j+1) - 2 + (p & (2^(j+1) - 1)), the state entering level j of each of the last
    2^(j+1) positions p (reference decoding.py:50-76, 143-185): the oracle scan run with j levels;
    beyond n_lv the final state. Slots of positions before the prompt stay untouched."""
    from dispatcher_hybrid import fused_gates as fg
    print(f"level_scan ring T={T} n_lv={n_lv} ring_L={ring_L}", flush=True)
    b, H, hd = 2, 2, 64
    rng = np.random.default_rng(T)
    pres = [rng.normal(size=(b, T, n_lv, H)) * 2 for _ in range(3)]
    V0 = rng.normal(size=(b, T, H * hd))
    mask = (rng.random((b, T, n_lv)) > 0.2).astype(np.float64)
    tp = [_cuda(p, torch.float32) for p in pres]
    tV0, tm = _cuda(V0, torch.float32), _cuda(mask, torch.float32)
    S = (2 << ring_L) - 2
    sentinel = -7.0
    ring = torch.full((b, S, H * hd), sentinel, device=DEV)
    out = torch.empty_like(tV0)
    fg._scan_launch(*tp, tm, tV0, out, H, n_lv, False, "test", ring=ring, ring_L=ring_L)
    torch.cuda.synchronize()
    got = ring.cpu().numpy()
    for j in range(ring_L):
        jj = min(j, n_lv)
        ref = V0 if jj == 0 else om.level_scan(*[p[:, :, :jj] for p in pres], V0, H, mask[..., :jj])
        span = 2 << j
        p0 = max(0, T - span)
        slots = (span - 2) + (np.arange(p0, T) & (span - 1))
        np.testing.assert_allclose(got[:, slots], ref[:, p0:T], rtol=1e-5, atol=1e-5)
        untouched = np.setdiff1d(np.arange(span - 2, 2 * span - 2), slots)
        assert np.all(got[:, untouched] == sentinel)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_level_scan_known_answers_exact(dtype):
    """Saturated gates with one-hot V0 rows: window sums / pure shifts are 0/1 vectors, which
    every dtype represents exactly, so the kernel must reproduce them bit for bit."""
    from dispatcher_hybrid.fused_gates import fused_level_scan
    T, H, hd = 128, 2, 64
    V0 = torch.zeros(1, T, H * hd, dtype=dtype, device=DEV)
    V0[0, torch.arange(T), torch.arange(T)] = 1
    for n_lv in (1, 3, 7):
        on = torch.full((1, T, n_lv, H), 30.0, dtype=dtype, device=DEV)
        off = torch.full((1, T, n_lv, H), -200.0, dtype=dtype, device=DEV)
        V = fused_level_scan(on, on, on, None, V0, H, n_lv)       # window sums of width 2^n_lv
        t = torch.arange(T, device=DEV)
        win = ((t[None, :] <= t[:, None]) & (t[None, :] > t[:, None] - (1 << n_lv))).to(dtype)
        assert torch.equal(V[0, :, :T], win)
        V = fused_level_scan(on, off, on, None, V0, H, n_lv)      # pure shift by 2^n_lv - 1
        src = (t - ((1 << n_lv) - 1)).clamp(min=0)
        assert torch.equal(V[0], V0[0, src])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_level_scan_known_answers_long_lags(dtype):
    """Lags of whole 1024-position slots (T = 4096: levels 10 and 11, lags 1024 and 2048) take their
    source from the thread's own registers instead of the LDS exchange. V0[t] = e_(t mod 128) with
    saturated gates: the window sums count each residue class's positions (at most 32, exact in
    every dtype) and the pure shifts move rows; both are checked bit for bit."""
    from dispatcher_hybrid.fused_gates import fused_level_scan
    T, H, hd = 4096, 2, 64
    C = H * hd
    t = torch.arange(T, device=DEV)
    V0 = torch.zeros(1, T, C, dtype=dtype, device=DEV)
    V0[0, t, t % C] = 1
    onehot = torch.zeros(T, C, device=DEV)
    onehot[t, t % C] = 1
    for n_lv in (11, 12):
        print(f"level_scan long lags n_lv={n_lv} dtype={dtype}", flush=True)
        on = torch.full((1, T, n_lv, H), 30.0, dtype=dtype, device=DEV)
        off = torch.full((1, T, n_lv, H), -200.0, dtype=dtype, device=DEV)
        V = fused_level_scan(on, on, on, None, V0, H, n_lv)       # window sums of width 2^n_lv
        win = ((t[None, :] <= t[:, None]) & (t[None, :] > t[:, None] - (1 << n_lv))).float()
        assert torch.equal(V[0], (win @ onehot).to(dtype))
        V = fused_level_scan(on, off, on, None, V0, H, n_lv)      # pure shift by 2^n_lv - 1
        src = (t - ((1 << n_lv) - 1)).clamp(min=0)
        assert torch.equal(V[0], V0[0, src])


# --------------------------------------------------------------------------------------------
# gate_scan_fwd: activated, masked gates written head-major by the pre-activation kernel, then the
# scan in its activated mode
# --------------------------------------------------------------------------------------------
GATE_SCAN_CASES = [
    # b, T, GH, H, hd, L, with_mask
    (1, 1, 64, 2, 16, 3, False),
    (2, 45, 64, 4, 16, 6, True),
    (1, 600, 128, 2, 32, 10, True),
    (3, 1024, 256, 16, 64, 11, True),    # C2 length and heads
    (2, 4096, 64, 2, 128, 12, True),     # full context
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", GATE_SCAN_CASES)
def test_gate_scan_matches_oracle(case, dtype):
    from dispatcher_hybrid.fused_gates import fused_gate_scan
    b, T, GH, H, hd, L, with_mask = case
    print(f"gate_scan case={case} dtype={dtype}", flush=True)
    rng = np.random.default_rng(hash(case) % 2**32)
    n_lv = om.active_levels(L, T)
    A = rng.normal(size=(b, T, GH)) * 0.7
    B = rng.normal(size=(b, T, GH)) * 0.7
    Ws = [rng.normal(size=(L, H, GH)) * 1.5 / np.sqrt(GH) for _ in range(3)]
    bs = [rng.normal(size=(L, H)) for _ in range(3)]
    V0 = rng.normal(size=(b, T, H * hd))
    mask = (rng.random((b, T, L)) > 0.25).astype(np.float64) if with_mask else None
    tA, tB, tV0 = _cuda(A, dtype), _cuda(B, dtype), _cuda(V0, dtype)
    tW = [_cuda(w, dtype) for w in Ws]
    tb = [_cuda(x, torch.float32) for x in bs]
    tm = None if mask is None else _cuda(mask, dtype)[..., :n_lv]
    V = fused_gate_scan(tA, tB, *tW, *tb, n_lv, tm, tV0, H)
    torch.cuda.synchronize()
    m = None if mask is None else mask[..., :n_lv]
    pre = om.gate_preacts(_np(tA), _np(tB), *[_np(w) for w in tW], *bs, n_lv, m)
    ref = om.level_scan(*pre, _np(tV0), H, m)
    err = rel_err(_np(V), ref)
    # bf16: pre-activations and sigmoid outputs rounded like the eager bf16 path, state in fp32
    assert err < (1e-5 if dtype == torch.float32 else 2e-2), f"rel {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b", [8, 5, 3, 1])
def test_activated_gates_release_widths(b, dtype):
    """The activated, masked, head-major gates (activate mode) against torch's sigmoid of the op's
    own pre-activations, at the released widths (GH 1024, 16 heads, 12 levels, T 4096) and batch
    sizes that select level groups of 4, 3, 2 and 1, then the full gate_scan against the two-op
    route. bf16 allows one rounding step of the sigmoid output."""
    from dispatcher_hybrid import fused_gates as fg
    print(f"activated gates b={b} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(40 + b)
    T, GH, H, hd, L = 4096, 1024, 16, 64, 12
    A = torch.randn(b, T, GH, device=DEV, generator=g).to(dtype)
    B = torch.randn(b, T, GH, device=DEV, generator=g).to(dtype)
    W = [(torch.randn(L, H, GH, device=DEV, generator=g) / GH ** 0.5).to(dtype) for _ in range(3)]
    bs = [torch.randn(L, H, device=DEV, generator=g) for _ in range(3)]
    mask = (torch.rand(b, T, L, device=DEV, generator=g) > 0.1).to(dtype)
    V0 = torch.randn(b, T, H * hd, device=DEV, generator=g).to(dtype)
    pre = fg.fused_gate_preacts(A, B, *W, *bs, L, mask)
    t = torch.arange(T, device=DEV).view(1, T, 1)
    M = ((t >= (1 << torch.arange(L, device=DEV)).view(1, 1, L)) & (mask > 0)).float().unsqueeze(-1)
    refs = (torch.sigmoid(pre[0].float()) * M, torch.sigmoid(pre[1].float()) * M + (1 - M),
            torch.sigmoid(pre[2].float()))
    ins = fg._prep_gate_inputs(A, B, *W, *bs, L)
    buf = torch.full((3, b, H, L, T), float("nan"), device=DEV, dtype=ins[0].dtype)
    gates = [buf[i].permute(0, 3, 2, 1) for i in range(3)]
    fg._preacts_launch(*ins, mask, gates, gates[0].stride(), 1, L, "test")
    torch.cuda.synchronize()
    tol = 1e-6 if dtype == torch.float32 else 2.0 ** -8
    for got, ref in zip(gates, refs):
        assert not bool(torch.isnan(got).any()), "unwritten gate entries"
        assert float((got.float() - ref).abs().max()) <= tol
    V1 = fg.fused_gate_scan(A, B, *W, *bs, L, mask, V0, H)
    V2 = fg.fused_level_scan(*pre, mask, V0, H, L)
    assert rel_err(V1, V2) < (1e-5 if dtype == torch.float32 else 2e-2)


def test_gate_scan_equals_two_op_path_fp32():
    """The head-major activated route and the reference-layout op route agree in fp32."""
    from dispatcher_hybrid.fused_gates import fused_gate_preacts, fused_gate_scan, fused_level_scan
    g = torch.Generator(device=DEV).manual_seed(4)
    b, T, GH, H, hd, L = 2, 777, 128, 4, 32, 10
    A = torch.randn(b, T, GH, device=DEV, generator=g)
    B = torch.randn(b, T, GH, device=DEV, generator=g)
    Ws = [torch.randn(L, H, GH, device=DEV, generator=g) / GH ** 0.5 for _ in range(3)]
    bs = [torch.randn(L, H, device=DEV, generator=g) for _ in range(3)]
    V0 = torch.randn(b, T, H * hd, device=DEV, generator=g)
    mask = (torch.rand(b, T, L, device=DEV, generator=g) > 0.3).float()
    V1 = fused_gate_scan(A, B, *Ws, *bs, L, mask, V0, H)
    V2 = fused_level_scan(*fused_gate_preacts(A, B, *Ws, *bs, L, mask), mask, V0, H, L)
    assert rel_err(V1, V2) < 1e-5


# --------------------------------------------------------------------------------------------
# decode step
# --------------------------------------------------------------------------------------------
class _DecodeState:
    def __init__(self, Bb, Tmax, GH, H, hd, L, dtype, sentinel=0.0):
        self.S = (2 << L) - 2
        d = H * hd
        self.B_hist = torch.zeros(Bb, Tmax, GH, dtype=dtype, device=DEV)
        self.rg_hist = torch.zeros(Bb, Tmax, L, H, dtype=dtype, device=DEV)
        self.V_ring = torch.full((Bb, self.S, d), sentinel, dtype=dtype, device=DEV)
        self.Y = torch.zeros(Bb, d, dtype=dtype, device=DEV)
        self.t_buf = torch.zeros(1, dtype=torch.long, device=DEV)


DECODE_CASES = [
    # B, T(steps), Tmax, GH, H, hd, L
    (1, 40, 64, 64, 2, 64, 6),
    (3, 70, 128, 128, 4, 16, 7),
    (16, 20, 64, 64, 2, 32, 6),
    (2, 24, 4096, 1024, 16, 64, 12),    # release shapes (first positions)
    (8, 30, 128, 256, 4, 32, 8),        # batched gate readouts (four rows per wave)
    (5, 24, 64, 128, 8, 16, 7),         # the same with a partial last group of rows
    (16, 20, 64, 128, 8, 16, 6),        # 128 (row, head) pairs: one row per mixer-step workgroup
]


def _run_decode(case, dtype, seed, split=False, W_zero=False, bias=None, V0_onehot=False, sentinel=0.0,
                two=False, out_proj=None):
    from dispatcher_hybrid import fused_step
    Bb, T, Tmax, GH, H, hd, L = case
    d = H * hd
    rng = np.random.default_rng(seed)
    A = rng.normal(size=(Bb, T, GH)) * 0.7
    Bs = rng.normal(size=(Bb, T, GH)) * 0.7
    V0 = rng.normal(size=(Bb, T, d))
    if V0_onehot:
        V0 = np.zeros((Bb, T, d))
        for b in range(Bb):
            V0[b, np.arange(T), (np.arange(T) + b) % d] = 1.0
    Ws = [(np.zeros((L, H, GH)) if W_zero else rng.normal(size=(L, H, GH)) / np.sqrt(GH)) for _ in range(3)]
    bs = [np.full((L, H), v) for v in bias] if bias is not None else [rng.normal(size=(L, H)) for _ in range(3)]
    tA, tBs, tV0 = _cuda(A, dtype), _cuda(Bs, dtype), _cuda(V0, dtype)
    tW = [_cuda(w, dtype) for w in Ws]
    tb = [_cuda(x, dtype) for x in bs]
    st = _DecodeState(Bb, Tmax, GH, H, hd, L, dtype, sentinel)
    IG = torch.zeros(Bb, L * H, dtype=torch.float32, device=DEV)
    FG = torch.zeros_like(IG)
    stage = torch.full((fused_step.stage_floats(Bb, H, L, hd),), float("nan"), device=DEV)
    Ys = []
    for t in range(T):
        st.B_hist[:, t] = tBs[:, t]
        st.t_buf.fill_(t)
        if split:
            fused_step.step_gates_kernel[(Bb, L)](tA[:, t].contiguous(), st.B_hist, *tW, *tb, st.t_buf,
                                                  IG, FG, st.rg_hist, Tmax, GH=GH, H=H, L=L, BK=128)
            fused_step.step_scan_kernel[(Bb, H)](tV0[:, t].contiguous(), IG, FG, st.rg_hist, st.V_ring,
                                                 st.t_buf, st.Y, Tmax, st.S, L=L, HD=hd, H=H)
        elif out_proj is not None:
            W_out, resid, outs = out_proj
            fused_step.decode_gates_scan_out(tA[:, t].contiguous(), st.B_hist, *tW, *tb, st.t_buf,
                                             st.rg_hist, st.V_ring, tV0[:, t].contiguous(), st.Y, stage,
                                             W_out, resid[t:t + 1], outs[t:t + 1])
        elif two:
            fused_step.decode_gates_scan(tA[:, t].contiguous(), st.B_hist, *tW, *tb, st.t_buf,
                                         st.rg_hist, st.V_ring, tV0[:, t].contiguous(), st.Y, stage)
        else:
            fused_step.decode_mixer_step(tA[:, t].contiguous(), st.B_hist, *tW, *tb, st.t_buf,
                                         st.rg_hist, st.V_ring, tV0[:, t].contiguous(), st.Y)
        Ys.append(st.Y.clone())
    torch.cuda.synchronize()
    inputs = dict(A=_np(tA), Bs=_np(tBs), V0=_np(tV0), W=[_np(w) for w in tW], b=[_np(x) for x in tb])
    return st, torch.stack(Ys, 1), inputs


def _oracle_decode(case, inp, sentinel=0.0):
    Bb, T, Tmax, GH, H, hd, L = case
    S = (2 << L) - 2
    rg = np.zeros((Bb, Tmax, L, H))
    ring = np.full((Bb, S, H * hd), sentinel)
    B_hist = np.zeros((Bb, Tmax, GH))
    Ys = []
    for t in range(T):
        B_hist[:, t] = inp["Bs"][:, t]
        Ys.append(om.decode_step(inp["A"][:, t], B_hist, *inp["W"], *inp["b"], t, rg, ring, inp["V0"][:, t]))
    return np.stack(Ys, 1), rg, ring


@pytest.mark.parametrize("two", [False, True], ids=["one_launch", "two_launches"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", DECODE_CASES)
def test_decode_mixer_step_matches_oracle(case, dtype, two):
    print(f"decode case={case} dtype={dtype} two={two}", flush=True)
    st, Y, inp = _run_decode(case, dtype, seed=11, two=two)
    Yo, rgo, ringo = _oracle_decode(case, inp)
    T = case[1]
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(_np(Y), Yo) < tol
    assert rel_err(_np(st.rg_hist[:, :T]), rgo[:, :T]) < (1e-6 if dtype == torch.float32 else 8e-3)
    assert rel_err(_np(st.V_ring), ringo) < tol


@pytest.mark.parametrize("two", [False, True], ids=["one_launch", "two_launches"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_ring_slots_bit_exact(dtype, two):
    """f = a = r = 1 (W = 0, biases +800) and one-hot V0 rows: every ring entry is a 0/1 window
    sum, exact in any dtype, and unwritten slots keep a sentinel. The whole ring, rg_hist and
    every output must equal the oracle's bit for bit."""
    case = (2, 100, 128, 64, 2, 64, 7)
    st, Y, inp = _run_decode(case, dtype, seed=3, W_zero=True, bias=(800.0, 800.0, 800.0),
                                V0_onehot=True, sentinel=-3.0, two=two)
    Yo, rgo, ringo = _oracle_decode(case, inp, sentinel=-3.0)
    assert np.array_equal(_np(st.V_ring), ringo)
    assert np.array_equal(_np(st.rg_hist), rgo)
    assert np.array_equal(_np(Y), Yo)


def test_split_launches_match_fused_kernel():
    """step_gates_kernel + step_scan_kernel (reference launch syntax) agree with one fused
    launch (different reduction trees: equal to rounding)."""
    case = (3, 30, 64, 128, 4, 16, 6)
    for dtype, tol in ((torch.float32, 1e-6), (torch.bfloat16, 2e-2)):
        a, Ya, _ = _run_decode(case, dtype, seed=5)
        b, Yb, _ = _run_decode(case, dtype, seed=5, split=True)
        assert rel_err(_np(Ya), _np(Yb)) < tol
        assert rel_err(_np(a.V_ring), _np(b.V_ring)) < tol
        assert rel_err(_np(a.rg_hist), _np(b.rg_hist)) < tol


@pytest.mark.parametrize("case", [(16, 12, 64, 1024, 16, 64, 12), (5, 20, 64, 64, 2, 128, 6),
                                  (2, 30, 64, 128, 4, 16, 7)])
def test_two_launch_step_equals_one_launch(case):
    """dh_decode_gates + dh_decode_scan against dh_decode_mixer_step: the same per-lane partial
    dot products, wave reductions and recurrence, so the outputs and caches agree to rounding
    (batch 16 takes the four-rows-per-wave gate path)."""
    for dtype, tol in ((torch.float32, 1e-6), (torch.bfloat16, 1e-2)):
        a, Ya, _ = _run_decode(case, dtype, seed=9)
        b, Yb, _ = _run_decode(case, dtype, seed=9, two=True)
        assert rel_err(_np(Ya), _np(Yb)) < tol
        assert rel_err(_np(a.V_ring), _np(b.V_ring)) < tol
        assert rel_err(_np(a.rg_hist), _np(b.rg_hist)) < tol


def test_decode_position_out_of_range_writes_nothing():
    from dispatcher_hybrid import fused_step
    Bb, Tmax, GH, H, hd, L = 2, 32, 64, 2, 64, 5
    st = _DecodeState(Bb, Tmax, GH, H, hd, L, torch.float32, sentinel=1.5)
    A = torch.randn(Bb, GH, device=DEV)
    W = torch.randn(L, H, GH, device=DEV)
    bias = torch.zeros(L, H, device=DEV)
    V0 = torch.randn(Bb, H * hd, device=DEV)
    before = (st.rg_hist.clone(), st.V_ring.clone(), st.Y.clone())
    for t in (Tmax, Tmax + 5, -1):
        st.t_buf.fill_(t)
        fused_step.decode_mixer_step(A, st.B_hist, W, W, W, bias, bias, bias, st.t_buf, st.rg_hist,
                                     st.V_ring, V0, st.Y)
    torch.cuda.synchronize()
    assert torch.equal(before[0], st.rg_hist) and torch.equal(before[1], st.V_ring)
    assert torch.equal(before[2], st.Y)


def test_decode_wrapper_rejects_mixed_dtypes():
    from dispatcher_hybrid import fused_step
    Bb, Tmax, GH, H, hd, L = 1, 16, 64, 2, 64, 4
    st = _DecodeState(Bb, Tmax, GH, H, hd, L, torch.float32)
    W = torch.randn(L, H, GH, device=DEV, dtype=torch.bfloat16)
    bias = torch.zeros(L, H, device=DEV)
    with pytest.raises(TypeError, match="dtype"):
        fused_step.decode_mixer_step(torch.randn(Bb, GH, device=DEV), st.B_hist, W, W, W, bias, bias,
                                     bias, st.t_buf, st.rg_hist, st.V_ring,
                                     torch.randn(Bb, H * hd, device=DEV), st.Y)


SCAN_OUT_CASES = [
    # B, T(steps), Tmax, GH, H, hd, L -- batch 1 (the fused recurrence + out-projection launch)
    (1, 40, 64, 64, 2, 64, 6),
    (1, 70, 128, 128, 4, 16, 7),
    (1, 24, 4096, 1024, 16, 64, 12),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", SCAN_OUT_CASES)
def test_scan_out_matches_two_launches_and_oracle(case, dtype):
    """dh_decode_gates + dh_decode_scan_out (the recurrence inside the out-projection launch) over T
    steps: Y, rg_hist and every ring slot equal the two-launch path's (same arithmetic, compared to
    one fp32 rounding), Y matches the oracle, and out = round(round(W_out . Y) + resid) matches a
    float64 product of the kernel's own Y (reference decoding.py:473-476)."""
    Bb, T, Tmax, GH, H, hd, L = case
    d = H * hd
    print(f"scan_out case={case} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T)
    W_out = (torch.randn(d, d, device=DEV, generator=g) / d ** 0.5).to(dtype)
    resid = torch.randn(T, d, device=DEV, generator=g).to(dtype)
    outs = torch.full((T, d), 5.0, device=DEV, dtype=dtype)
    a, Ya, inp = _run_decode(case, dtype, seed=13, two=True)
    b, Yb, _ = _run_decode(case, dtype, seed=13, out_proj=(W_out, resid, outs))
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert rel_err(_np(Yb), _np(Ya)) < tol
    assert rel_err(_np(b.V_ring), _np(a.V_ring)) < tol
    assert torch.equal(b.rg_hist, a.rg_hist)
    Yo, _, _ = _oracle_decode(case, inp)
    assert rel_err(_np(Yb), Yo) < (1e-4 if dtype == torch.float32 else 2e-2)
    rnd = (lambda x: x.to(dtype).double()) if dtype == torch.bfloat16 else (lambda x: x)
    ref = rnd(rnd(Yb[0].double() @ W_out.double().T) + resid.double())
    assert rel_err(outs.double(), ref) < (1e-5 if dtype == torch.float32 else 1e-2)


def test_scan_out_residual_rows_in_place_and_range():
    """The residual read through resid_rows (the first layer's embedding row), `out` aliasing the
    residual row, and a position outside [0, Tmax) writing nothing."""
    from dispatcher_hybrid import fused_step
    Bb, Tmax, GH, H, hd, L = 1, 64, 64, 2, 64, 6
    d = H * hd
    g = torch.Generator(device=DEV).manual_seed(31)
    st = _DecodeState(Bb, Tmax, GH, H, hd, L, torch.float32, 0.0)
    A = torch.randn(1, GH, device=DEV, generator=g)
    V0 = torch.randn(1, d, device=DEV, generator=g)
    Ws = [torch.randn(L, H, GH, device=DEV, generator=g) / 8 for _ in range(3)]
    bs = [torch.randn(L, H, device=DEV, generator=g) for _ in range(3)]
    W_out = torch.randn(d, d, device=DEV, generator=g) / d ** 0.5
    emb = torch.randn(50, d, device=DEV, generator=g)
    rows = torch.tensor([37], device=DEV)
    x = torch.zeros(1, d, device=DEV)
    stage = torch.zeros(fused_step.stage_floats(1, H, L, hd), device=DEV)
    st.B_hist[:, 5] = torch.randn(GH, device=DEV, generator=g)
    st.t_buf.fill_(5)
    fused_step.decode_gates_scan_out(A, st.B_hist, *Ws, *bs, st.t_buf, st.rg_hist, st.V_ring, V0, st.Y, stage,
                                      W_out, emb, x, resid_rows=rows)
    torch.cuda.synchronize()
    assert rel_err(x, st.Y.double() @ W_out.double().T + emb[37].double()) < 1e-5
    x2 = emb[3:4].clone()
    fused_step.decode_gates_scan_out(A, st.B_hist, *Ws, *bs, st.t_buf, st.rg_hist, st.V_ring, V0, st.Y, stage,
                                      W_out, x2, x2)                     # in place
    torch.cuda.synchronize()
    assert rel_err(x2, st.Y.double() @ W_out.double().T + emb[3].double()) < 1e-5
    ring0, Y0, x3 = st.V_ring.clone(), st.Y.clone(), x.clone()
    st.t_buf.fill_(Tmax)
    fused_step.decode_gates_scan_out(A, st.B_hist, *Ws, *bs, st.t_buf, st.rg_hist, st.V_ring, V0, st.Y, stage,
                                      W_out, emb, x, resid_rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(st.V_ring, ring0) and torch.equal(st.Y, Y0) and torch.equal(x, x3)


# ---- dh_silu_mul: the SwiGLU activation (reference modeling_dispatcher.py:197) ----

def _bf16_round_np(x):
    """fp32 -> bf16 -> fp32, round to nearest even (numpy, the CPU statement of the rounding)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 4096 + 5, 1024 * 2816 + 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_silu_mul_matches_eager_swiglu(n, dtype):
    from dispatcher_hybrid.fused_gates import silu_mul
    g = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 4).to("cuda", dtype)
    u = torch.randn(n, generator=torch.Generator().manual_seed(n + 1)).to("cuda", dtype)
    out = silu_mul(g, u)
    ref = torch.nn.functional.silu(g) * u          # the reference's eager activation
    # CPU statement of the same rounding points in float64 math
    g64, u64 = _np(g).astype(np.float64), _np(u).astype(np.float64)
    s = g64 / (1.0 + np.exp(-g64))
    if dtype == torch.bfloat16:
        cpu = _bf16_round_np(_bf16_round_np(s.astype(np.float32)).astype(np.float64) * u64)
        # bit-exact against torch's kernel: the bf16 silu equals torch's for every bf16 input (see
        # test_silu_mul_bf16_every_input) and the product of two bf16 values is exact in fp32
        assert torch.equal(out, ref)
        dc = np.abs(_np(out).astype(np.float64) - cpu)
        assert (dc <= np.maximum(np.abs(cpu), 1e-30) * 2.0 ** -7).all()
    else:
        assert rel_err(_np(out), _np(ref)) <= 1e-6 if n else True
        if n:
            assert np.allclose(_np(out), s * u64, rtol=2e-6, atol=1e-30)


def test_silu_mul_bf16_every_input():
    """All 65536 bf16 gate patterns (NaN aside) with up = 1: dh_silu_mul's bf16 activation (silu with
    the hardware exp and an IEEE divide, then the product) equals torch's bf16 SiLU bit for bit, so
    the faster exp never moves a rounded result (the fused SwiGLU GEMM epilogue evaluates the same)."""
    from dispatcher_hybrid.fused_gates import silu_mul
    g = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).to("cuda")
    u = torch.ones(65536, device="cuda", dtype=torch.bfloat16)
    out = silu_mul(g, u)
    ref = torch.nn.functional.silu(g) * u
    keep = ~torch.isnan(g.float())
    assert int(keep.sum()) == 65536 - 254
    rn = torch.isnan(ref.float())                    # silu(-inf) = -inf / inf: a NaN (of either sign)
    assert torch.equal(torch.isnan(out.float())[keep], rn[keep])
    num = keep & ~rn
    assert torch.equal(out.view(torch.int16)[num], ref.view(torch.int16)[num])


def test_silu_mul_in_place_and_unaligned_views():
    from dispatcher_hybrid.fused_gates import silu_mul
    base_g = torch.randn(10001, device="cuda", dtype=torch.bfloat16)
    base_u = torch.randn(10001, device="cuda", dtype=torch.bfloat16)
    g, u = base_g[1:], base_u[1:]                 # 2-byte storage offset: copied by the wrapper
    want = silu_mul(g.clone(), u.clone())
    assert torch.equal(silu_mul(g, u), want)
    gi = g.clone()
    got = silu_mul(gi, u.clone(), out=gi)          # in place over gate, as SwiGLU's fused forward does
    assert got.data_ptr() == gi.data_ptr() and torch.equal(got, want)
    with pytest.raises(ValueError):
        silu_mul(g, u.float())


# ---- dh_add_rmsnorm: residual add + the RMSNorm after it (reference modeling_dispatcher.py:210-212) ----

@pytest.mark.parametrize("rows,d", [(0, 1024), (1, 1024), (7, 1024), (1030, 1024), (5, 776), (3, 8), (9, 4096),
                                    (2, 8192)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_add_rmsnorm_matches_eager_add_and_norm(rows, d, dtype):
    from dispatcher_hybrid.fused_gates import add_rmsnorm
    if dtype == torch.float32 and d > 4096:
        pytest.skip("fp32 rows are limited to 4096 elements")
    gen = torch.Generator().manual_seed(rows * 7 + d)
    x = (torch.randn(rows, d, generator=gen) * 3).to("cuda", dtype)
    y = torch.randn(rows, d, generator=gen).to("cuda", dtype)
    norm = torch.nn.RMSNorm(d).to("cuda", dtype)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(d, generator=gen) + 0.5)
        s_ref = x + y                                   # the eager residual add
        h_ref = norm(s_ref)                             # the eager RMSNorm (eps None: fp32 epsilon)
        xo, h = add_rmsnorm(x, y, norm)
    assert torch.equal(xo, s_ref)                       # the sum: same rounding, bit-exact
    # the norm in fp64 from the (exact) bf16/fp32 sum: a reduction-order-free statement of the formula
    s64 = s_ref.double()
    truth = s64 * torch.rsqrt((s64 * s64).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps) * norm.weight.double()
    if rows == 0:
        assert h.shape == (0, d)
        return
    if dtype == torch.bfloat16:
        tol = truth.abs() * 2.0 ** -8 + 1e-30         # half a bf16 ulp of rounding + fp32 noise
        assert bool(((h.double() - truth).abs() <= tol * 1.01).all())
        # and against torch's kernel: at most one bf16 ulp apart, rarely
        d_ = (h.float() - h_ref.float()).abs()
        assert bool((d_ <= h_ref.float().abs() * 2.0 ** -7 + 1e-30).all())
        assert int((d_ > 0).sum()) <= max(2, h.numel() // 500)
    else:
        assert rel_err(h, truth) <= 2e-6
        assert rel_err(h, h_ref) <= 2e-6


def test_add_rmsnorm_in_place_and_errors():
    from dispatcher_hybrid.fused_gates import add_rmsnorm
    x = torch.randn(64, 1024, device="cuda", dtype=torch.bfloat16)
    y = torch.randn(64, 1024, device="cuda", dtype=torch.bfloat16)
    norm = torch.nn.RMSNorm(1024, eps=1e-5).to("cuda", torch.bfloat16)
    with torch.no_grad():
        want_x, want_h = add_rmsnorm(x, y, norm)
        xi = x.clone()
        got_x, got_h = add_rmsnorm(xi, y, norm, out=xi)   # the fused block loop writes the sum over x
        assert got_x.data_ptr() == xi.data_ptr()
        assert torch.equal(got_x, want_x) and torch.equal(got_h, want_h)
        with pytest.raises(ValueError):
            add_rmsnorm(x, y.float(), norm)
        with pytest.raises(ValueError):
            add_rmsnorm(x, y, torch.nn.RMSNorm(1024).to("cuda"))   # fp32 weight with bf16 rows


# --------------------------------------------------------------------------------------------
# tree mask with document resets
# --------------------------------------------------------------------------------------------
TREE_MASK_CASES = [
    # b, T, L, eot placement
    (1, 1, 3, "none"),
    (3, 5, 12, "random"),               # levels whose lag is >= T stay all zero
    (2, 37, 6, "edges"),                # EOT at the first and the last position
    (2, 1025, 11, "random"),            # one position past a multiple of the 1024 threads
    (4, 4096, 12, "random"),            # C2/C5 row length
    (2, 4096, 12, "dense"),             # every other token an EOT
    (1, 16384, 14, "random"),           # the longest row the kernel takes
]


def _tree_ids(case, eot=7):
    b, T, L, kind = case
    rng = np.random.default_rng(T * 31 + b)
    ids = rng.integers(0, 50, size=(b, T))
    ids[ids == eot] = eot + 1
    if kind == "random":
        ids[rng.random((b, T)) < 8.0 / T + 0.003] = eot
        if b > 1:
            ids[-1] = eot               # an all-EOT row
        if b > 2:
            ids[1] = eot + 1            # a row without one
    elif kind == "edges":
        ids[:, 0] = eot
        ids[:, -1] = eot
    elif kind == "dense":
        ids[:, ::2] = eot
    return ids, eot


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", TREE_MASK_CASES)
def test_tree_mask_equals_oracle(case, dtype):
    """dh_tree_mask's 0/1 values bit-exact against the oracle's tree_mask (level mask x doc reset)."""
    from dispatcher_hybrid.fused_gates import tree_mask
    print(f"tree_mask case={case} dtype={dtype}", flush=True)
    ids, eot = _tree_ids(case)
    L = case[2]
    got = tree_mask(torch.as_tensor(ids, dtype=torch.int64, device=DEV), L, eot, dtype)
    assert got.shape == (*ids.shape, L) and got.dtype == dtype and got.is_contiguous()
    ref = torch.as_tensor(om.tree_mask(ids, L, eot)).to(dtype)
    assert torch.equal(got.cpu(), ref)


def test_tree_mask_strided_ids_and_rejects():
    """A row-strided view of the ids (a slice of a wider batch) reads the right rows; shapes and
    dtypes outside the kernel's range raise before any launch."""
    from dispatcher_hybrid.fused_gates import tree_mask
    ids, eot = _tree_ids((3, 300, 9, "random"))
    wide = torch.zeros(3, 512, dtype=torch.int64, device=DEV)
    wide[:, 100:400] = torch.as_tensor(ids, device=DEV)
    view = wide[:, 100:400]
    assert view.stride(0) == 512
    got = tree_mask(view, 9, eot, torch.float32)
    assert torch.equal(got.cpu(), torch.as_tensor(om.tree_mask(ids, 9, eot)).float())
    # an expanded batch (row stride 0) is read as the repeated row
    one = torch.as_tensor(ids[:1], dtype=torch.int64, device=DEV).expand(3, -1)
    got = tree_mask(one, 9, eot, torch.bfloat16)
    assert torch.equal(got.cpu(), torch.as_tensor(om.tree_mask(np.repeat(ids[:1], 3, 0), 9, eot)).to(torch.bfloat16))
    t = torch.as_tensor(ids, device=DEV)
    with pytest.raises(ValueError):
        tree_mask(t.to(torch.int32), 9, eot, torch.float32)
    with pytest.raises(ValueError):
        tree_mask(t, 9, eot, torch.float16)
    with pytest.raises(ValueError):
        tree_mask(t, 31, eot, torch.float32)
    with pytest.raises(ValueError):
        tree_mask(torch.zeros(1, 16385, dtype=torch.int64, device=DEV), 9, eot, torch.float32)
