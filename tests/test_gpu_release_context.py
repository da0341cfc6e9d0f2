"""Decode parity at the released context: L = 12 levels, positions t >= 2048 (level 11 live, ring 11
read), the 4096-token context the C3 and C4 workloads decode at.

Reference contracts restated here:
  eager tree step                 dispatcher_hybrid/decoding.py:187-222
  ring slots / recurrence         dispatcher_hybrid/fused_step.py:62-88
  fused decoder = parallel/eager  tests/test_decoding.py:47-58
  ring layout                     tests/test_decoding.py:121-131
  batched = solo                  tests/test_decoding.py:134-153
  batched graphed/fused (bf16)    tests/test_decoding.py:156-178
"""

import numpy as np
import pytest
import torch

from dispatcher_hybrid.numerics import fp32_product_accumulation
from helpers import bf16_vs_truth, preact_bound, product_model, rel_err
from oracle import mixer as om
from test_gpu_kernels import _np, _oracle_decode, _run_decode
from weights import RELEASE_CONFIG, make_state_dict

pytestmark = pytest.mark.gpu
DEV = "cuda"

GH, H, HD, L, TMAX = 1024, 16, 64, 12, 4096
POSITIONS = [2047, 2048, 3000, 3899, 4095]


# --------------------------------------------------------------------------------------------
# kernel level: one step at a late position from a state the oracle fills
# --------------------------------------------------------------------------------------------
def _late_state(Bb, dtype, seed):
    """A decode state as a run up to any position < TMAX could have left it: every B_hist row, every
    transmit gate and every ring slot drawn at random (rounded to `dtype`), plus this step's A, V0,
    gate weights and biases."""
    rng = np.random.default_rng(seed)
    d = H * HD
    S = (2 << L) - 2
    rnd = lambda a: torch.as_tensor(a, dtype=torch.float64).to(dtype).double().numpy()
    return dict(
        B_hist=rnd(rng.normal(size=(Bb, TMAX, GH)) * 0.7),
        rg=rnd(rng.uniform(0.05, 0.95, size=(Bb, TMAX, L, H))),
        ring=rnd(rng.normal(size=(Bb, S, d))),
        A=rnd(rng.normal(size=(Bb, GH)) * 0.7),
        V0=rnd(rng.normal(size=(Bb, d))),
        W=[rnd(rng.normal(size=(L, H, GH)) / np.sqrt(GH)) for _ in range(3)],
        b=[rnd(rng.normal(size=(L, H))) for _ in range(3)])


@pytest.mark.parametrize("t", POSITIONS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("path", ["scan_out_b1", "gates_scan_b2"])
def test_release_step_at_late_position_matches_oracle(path, dtype, t):
    """dh_decode_gates + dh_decode_scan_out (batch 1, the graphed step's tree layer) and
    dh_decode_gates + dh_decode_scan (batch 2) at release widths against the float64 oracle: Y, the
    transmit gates written at t, and the whole ring (the slot of t at every level written, every
    other slot untouched)."""
    from dispatcher_hybrid import fused_step
    Bb = 1 if path == "scan_out_b1" else 2
    print(f"late step path={path} dtype={dtype} t={t}", flush=True)
    st = _late_state(Bb, dtype, seed=t)
    cu = lambda a: torch.as_tensor(a).to(DEV, dtype).contiguous()
    B_hist, rg_hist, V_ring = cu(st["B_hist"]), cu(st["rg"]), cu(st["ring"])
    A, V0 = cu(st["A"]), cu(st["V0"])
    W = [cu(w) for w in st["W"]]
    b = [cu(x) for x in st["b"]]
    d = H * HD
    Y = torch.full((Bb, d), float("nan"), device=DEV, dtype=dtype)
    t_buf = torch.full((1,), t, dtype=torch.long, device=DEV)
    stage = torch.full((fused_step.stage_floats(Bb, H, L, HD),), float("nan"), device=DEV)
    if path == "scan_out_b1":
        g = torch.Generator(device=DEV).manual_seed(t)
        W_out = (torch.randn(d, d, device=DEV, generator=g) / d ** 0.5).to(dtype)
        resid = torch.randn(1, d, device=DEV, generator=g).to(dtype)
        out = torch.empty(1, d, device=DEV, dtype=dtype)
        fused_step.decode_gates_scan_out(A, B_hist, *W, *b, t_buf, rg_hist, V_ring, V0, Y, stage, W_out, resid, out)
    else:
        fused_step.decode_gates_scan(A, B_hist, *W, *b, t_buf, rg_hist, V_ring, V0, Y, stage)
    torch.cuda.synchronize()
    rg_o, ring_o = st["rg"].copy(), st["ring"].copy()
    Yo = om.decode_step(st["A"], st["B_hist"], *st["W"], *st["b"], t, rg_o, ring_o, st["V0"])
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(_np(Y), Yo) < tol
    assert rel_err(_np(rg_hist[:, t]), rg_o[:, t]) < (1e-6 if dtype == torch.float32 else 8e-3)
    ring = _np(V_ring)
    written = np.array([om.ring_slot(j, t) for j in range(L)])
    keep = np.setdiff1d(np.arange(ring.shape[1]), written)
    assert np.array_equal(ring[:, keep], ring_o[:, keep]), "a slot other than t's was written"
    assert rel_err(ring[:, written], ring_o[:, written]) < tol
    other = np.setdiff1d(np.arange(TMAX), [t])
    assert np.array_equal(_np(rg_hist[:, other]), st["rg"][:, other]), "rg_hist written outside row t"
    if path == "scan_out_b1":
        ref = (Y[0].double() @ W_out.double().T) + resid.double()
        assert rel_err(out.double(), ref) < (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("two", [True, False], ids=["gates_scan", "gates_scan_out"])
def test_release_ring_kat_every_position_to_4096(dtype, two):
    """Saturated gates (W = 0, biases +800: f = a = r = 1) and one-hot V0 rows, L = 12, every position
    0 .. 4095: each ring entry and output is an integer window count (at most 64 here), exact in
    bf16, so the whole ring, rg_hist and every Y must equal the oracle's bit for bit; unwritten
    slots keep their sentinel."""
    case = (1, TMAX, TMAX, 64, 1, 64, L)
    out_proj = None
    if not two:
        out_proj = (torch.zeros(64, 64, device=DEV, dtype=dtype), torch.zeros(TMAX, 64, device=DEV, dtype=dtype),
                    torch.empty(TMAX, 64, device=DEV, dtype=dtype))
    print(f"ring KAT L=12 dtype={dtype} two={two}", flush=True)
    st, Y, inp = _run_decode(case, dtype, seed=3, W_zero=True, bias=(800.0, 800.0, 800.0), V0_onehot=True,
                             sentinel=-3.0, two=two, out_proj=out_proj)
    Yo, rgo, ringo = _oracle_decode(case, inp, sentinel=-3.0)
    assert np.array_equal(_np(st.V_ring), ringo)
    assert np.array_equal(_np(st.rg_hist), rgo)
    assert np.array_equal(_np(Y), Yo)
    assert Yo.max() == 64.0                                 # t = 4095: 4096 positions over 64 columns


# --------------------------------------------------------------------------------------------
# model level: the released 292M architecture (random init)
# --------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def release():
    """292M random init (reference scheme, W1s ~ N(0, 0.02) so every lag's source row matters), fp32
    and bf16 on the GPU."""
    cfgd = RELEASE_CONFIG
    sd = make_state_dict(cfgd, 0, scheme="reference")
    g = torch.Generator().manual_seed(1)
    for k in list(sd):
        if k.endswith("gate_hidden_src.weight"):
            sd[k] = torch.randn(sd[k].shape, generator=g) * 0.02
    m32 = product_model(cfgd, sd, device=DEV)
    m16 = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16)
    return cfgd, m32, m16


def _teacher_forced(dec, prompt, toks):
    """Logits of dec after prefill(prompt) for each step fed toks[:, j]: (B, n, V) fp32."""
    dec.prefill(prompt)
    return torch.stack([dec.step(toks[:, j]).float() for j in range(toks.shape[1])], 1)


def test_release_decode_at_4096_context(release):
    """C3 context: prefill 3840, then 64 steps (t = 3840 .. 3903) and a second decoder from a
    4032-token prompt to the last position (t = 4032 .. 4095). fp32: the fused decoder (graph of
    launches) against the fp32 eager decoder, rel <= 1e-4 and equal argmax. bf16: the one-launch
    greedy step's logits against the eager decoders teacher-forced with its own tokens."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    cfgd, m32, m16 = release
    g = torch.Generator(device=DEV).manual_seed(3)
    for P, n in ((3840, 64), (4032, 64)):
        ids = torch.randint(0, cfgd["vocab_size"] - 1, (1, P + n), device=DEV, generator=g)
        print(f"C3 fp32 prompt={P} steps={n}", flush=True)
        e32 = _teacher_forced(IncrementalDecoder(m32), ids[:, :P], ids[:, P:])
        f32 = _teacher_forced(FusedGraphedHybridDecoder(m32), ids[:, :P], ids[:, P:])
        r = rel_err(f32, e32)
        print(f"C3 fp32 prompt={P}: fused vs eager rel={r:.2e}", flush=True)
        assert r <= 1e-4
        assert bool((f32.argmax(-1) == e32.argmax(-1)).all())

        print(f"C3 bf16 one-launch greedy prompt={P} steps={n}", flush=True)
        dp = FusedGraphedHybridDecoder(m16)
        dp.greedy_start(dp.prefill(ids[:, :P])[:, -1])
        logits = []
        for _ in range(n):
            dp.step_greedy()
            logits.append(dp.logits_out.float().clone())
        assert dp._pers, "the one-launch step must have run"
        assert dp.check_persistent() == 0
        got = torch.stack(logits, 1)
        toks = dp.tok_hist[:, P:P + n]                       # the tokens fed to steps P .. P+n-1
        e16 = _teacher_forced(IncrementalDecoder(m16), ids[:, :P], toks)
        with fp32_product_accumulation():
            a16 = _teacher_forced(IncrementalDecoder(m16), ids[:, :P], toks)
        t32 = _teacher_forced(IncrementalDecoder(m32), ids[:, :P], toks)
        bf16_vs_truth(got, e16, t32, f"C3 bf16 prompt={P}", alt16=a16)


@pytest.mark.parametrize("P", [2040, 4070])
def test_release_one_launch_equals_graph_across_level_11(release, P):
    """The one-launch step and the graph of launches bit for bit (logits, tokens, every state
    buffer) across t = 2047 .. 2056, where level 11's first source appears, and up to t = 4095."""
    from test_gpu_persistent import _pair, _run_and_compare
    cfgd, _, m16 = release
    prompt = torch.randint(0, cfgd["vocab_size"] - 1, (1, P), device=DEV,
                           generator=torch.Generator(device=DEV).manual_seed(P))
    steps = min(26, TMAX - P)
    print(f"one-launch vs graph prompt={P} steps={steps}", flush=True)
    dp, dg = _pair(m16, prompt)
    _run_and_compare(dp, dg, steps)


def test_release_batch16_decode(release):
    """C4 shape: 16 rows sharing a 2048-token prefix, each continued with its own tokens for 8
    steps. fp32: rows of the batched fused decoder equal solo eager runs (rel <= 1e-4). bf16: the
    batched fused decoder (matrix-core batch GEMVs) against the fp32 eager decoder, and the device
    top-k sampler at B = 16 draws only inside each row's top-50 (temperature 0.8)."""
    from dispatcher_hybrid import fused_step
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    cfgd, m32, m16 = release
    g = torch.Generator(device=DEV).manual_seed(4)
    V = cfgd["vocab_size"]
    prefix = torch.randint(0, V - 1, (1, 2048), device=DEV, generator=g).expand(16, -1).contiguous()
    nexts = torch.randint(0, V - 1, (16, 8), device=DEV, generator=g)
    print("C4 fp32 batched vs solo", flush=True)
    b32 = _teacher_forced(FusedGraphedHybridDecoder(m32), prefix, nexts)
    for r in (0, 7, 15):
        solo = _teacher_forced(IncrementalDecoder(m32), prefix[r:r + 1], nexts[r:r + 1])
        rr = rel_err(b32[r:r + 1], solo)
        print(f"C4 fp32 row {r}: batched fused vs solo eager rel={rr:.2e}", flush=True)
        assert rr <= 1e-4
    print("C4 bf16 batched vs fp32 eager", flush=True)
    dec = FusedGraphedHybridDecoder(m16)
    f16 = _teacher_forced(dec, prefix, nexts)
    e16 = _teacher_forced(IncrementalDecoder(m16), prefix, nexts)
    t32 = _teacher_forced(IncrementalDecoder(m32), prefix, nexts)
    bf16_vs_truth(f16, e16, t32, "C4 bf16 B=16")
    lg = f16[:, -1].contiguous()
    kth = torch.topk(lg, 50, dim=-1).values[:, -1:]
    for seed in range(8):
        tok = fused_step.sample_tokens(lg, temperature=0.8, top_k=50, seed=seed)
        assert bool((lg.gather(1, tok[:, None]) >= kth).all()), f"draw outside the top-50 (seed {seed})"


def test_release_gate_preacts_c5_every_tree_layer(release):
    """C5 shape (B = 8, T = 4096, 12 levels, EOTs planted so the doc-reset mask is in play): the fused
    op's pre-activations of every tree layer against the eager formula on the same bf16 A and B
    (reference modeling_dispatcher.py:100-109), bounded in bf16 ulps at the eager rounding points
    (helpers.preact_bound: half an ulp of the eager product's rounding, half an ulp of each side's
    final rounding, plus the fp32 accumulation-order term). The share of values within the north
    star's 3e-2 is printed beside it."""
    from dispatcher_hybrid.modeling_dispatcher import level_gate_matmul
    cfgd, _, m16 = release
    g = torch.Generator(device=DEV).manual_seed(6)
    ids = torch.randint(0, cfgd["vocab_size"], (8, 4096), device=DEV, generator=g)
    for r in range(8):
        ids[r, 300 + 450 * r] = cfgd["eot_token"]
        ids[r, 3500 - 97 * r] = cfgd["eot_token"]
    caps = []
    mixers = [blk.mixer for blk in m16.blocks if hasattr(blk, "mixer")]
    hooks = [mx.register_forward_pre_hook(lambda mod, inp: caps.append(inp)) for mx in mixers]
    try:
        with torch.no_grad():
            m16(ids)
    finally:
        for hk in hooks:
            hk.remove()
    assert len(caps) == len(mixers) == 16
    worst = worst_abs = 0.0
    for li, (mx, (x, mask)) in enumerate(zip(mixers, caps)):
        with torch.no_grad():
            A, Bs = mx.gate_hidden(x), mx.gate_hidden_src(x)
            n_lv = 12
            m3 = mask[..., :n_lv]
            assert float(m3.sum()) < 8 * 4096 * n_lv - 8 * 4095    # the doc mask removes edges
            fused = torch.ops.dispatcher.gate_preacts_fwd(A, Bs, mx.gate_out, mx.forget_out, mx.reset_out,
                                                          mx.gate_out_bias, mx.forget_out_bias,
                                                          mx.reset_out_bias, n_lv, m3)
            lagged = torch.stack([torch.roll(Bs, shifts=1 << l, dims=1) for l in range(n_lv)], dim=2)
            hidden = torch.relu(A.unsqueeze(2) + lagged * m3.unsqueeze(-1)) ** 2
            del lagged
            for got, (W, b) in zip(fused, mx._gate_params()):
                ref = level_gate_matmul(hidden, W[:n_lv]) + b[:n_lv]
                bound = preact_bound(got, ref, b[:n_lv].float().expand_as(ref), level_gate_matmul(hidden, W[:n_lv].abs()))
                diff = (got.float() - ref.float()).abs()
                ratio = (diff / bound).max().item()
                worst = max(worst, ratio)
                within = (diff <= 3e-2).double().mean().item()
                worst_abs = max(worst_abs, diff.max().item())
                assert ratio <= 1.0, f"tree layer {li}: |d|/bound {ratio:.3f}"
                assert within >= 0.999, f"tree layer {li}: only {within:.5f} within 3e-2"
            del hidden, fused
    print(f"C5 gate preacts, 16 tree layers: worst |d|/ulp-bound {worst:.3f}, max |d| {worst_abs:.4f}", flush=True)
