"""Pins the oracle (oracle/) before it is trusted as the checker of the HIP kernels.

Each oracle function is checked against something other than its own formula:
  ring_slot / ring_offset   brute-force disjointness and no write/read collision over the release
                            shape; numpy restatement
  level_mask / tree_mask    closed form; the reference's own _tree_mask output (golden)
  gate_preacts              an independent numpy formulation (np.roll + matmul, a library routine);
                            the B = 0 special case that reduces to relu(A)^2 @ W^T; the reference's
                            mixer output at the release shape (golden)
  level_scan                closed forms with saturated gates: f=a=r=1 gives window sums and, after
                            every level, the causal prefix sum; f=0, a=r=1 gives a pure shift
  decode_step               the decoder == parallel identity (every step's output and every live
                            ring slot equals the parallel scan state), plus the reference's own
                            eager decoder state (golden)
  torch_eager               the reference's logits, decoder logits/state and greedy tokens (golden)
Plants: each pin is shown to fail on a deliberately wrong oracle variant (wrong lag, transposed
operand, dropped forget term), planted in the oracle inputs on the CPU.
"""

import numpy as np
import pytest
import torch

from helpers import golden, max_abs, rel_err, tiny
from oracle import mixer as om
from oracle import torch_eager as te
from weights import RELEASE_CONFIG, TINY_CONFIGS, checksum, make_state_dict, mixer_state_dict


# --------------------------------------------------------------------------------------------
# ring arithmetic
# --------------------------------------------------------------------------------------------
def test_ring_layout_release_shape():
    L, Tmax = 12, 4096
    S = (1 << (L + 1)) - 2
    assert S == 8190
    # ring j's slot range is contiguous, starts where ring j-1 ends, and the last ends at S
    end = 0
    for j in range(L):
        lo = om.ring_offset(j)
        assert lo == end
        slots = {om.ring_slot(j, p) for p in range(1 << (j + 1))}
        assert slots == set(range(lo, lo + (1 << (j + 1))))
        end = lo + (1 << (j + 1))
    assert end == S
    # the slot written at t never aliases the slot read at t - 2^l (same ring), for every t, l
    t = np.arange(Tmax)
    for l in range(L):
        w = om.ring_slots_numpy(l, t)
        r = om.ring_slots_numpy(l, np.maximum(t - (1 << l), 0))
        assert np.all((w != r) | (t < (1 << l)))
        # C and numpy agree
        for p in (0, 1, 2, 3, 1000, 4095):
            assert om.ring_slot(l, p) == int(om.ring_slots_numpy(l, p))
    # last 2^(j+1) positions occupy distinct slots (what write_slab relies on)
    for j in range(L):
        p = np.arange(Tmax - (1 << (j + 1)), Tmax)
        assert len(set(om.ring_slots_numpy(j, p).tolist())) == len(p)


# --------------------------------------------------------------------------------------------
# masks
# --------------------------------------------------------------------------------------------
def test_level_mask_closed_form():
    m = om.level_mask(10, 5)
    for t in range(10):
        for l in range(5):
            assert m[t, l] == (1.0 if (t >= 2 ** l and 2 ** l < 10) else 0.0)


@pytest.mark.parametrize("name", sorted(TINY_CONFIGS))
def test_tree_mask_matches_reference(name):
    g = golden(name)
    cfgd = TINY_CONFIGS[name]
    L = int(np.log2(cfgd["max_len"]))
    got = om.tree_mask(g["ids"], L, cfgd["eot_token"])
    assert np.array_equal(got, g["tree_mask"])
    spec = te.Spec(type("C", (), cfgd))
    got_t = te.tree_mask(spec, torch.from_numpy(g["ids"]), torch.float32)
    assert np.array_equal(got_t.numpy(), g["tree_mask"])


# --------------------------------------------------------------------------------------------
# gate pre-activations
# --------------------------------------------------------------------------------------------
def _numpy_preacts(A, B, W, b, n_lv, mask):
    """Independent formulation: lagged copies by np.roll, masked, relu^2, library matmul."""
    nb, T, GH = A.shape
    outs = []
    for l in range(n_lv):
        lag = np.roll(B, 1 << l, axis=1)
        open_ = (np.arange(T) >= (1 << l))[None, :, None].astype(np.float64)
        if mask is not None:
            open_ = open_ * (mask[:, :, l:l + 1] > 0)
        hid = np.maximum(A + lag * open_, 0.0) ** 2
        outs.append(hid @ W[l].T + b[l])              # (nb, T, H)
    return np.stack(outs, axis=2)


@pytest.mark.parametrize("with_mask", [False, True])
def test_gate_preacts_vs_numpy(with_mask):
    rng = np.random.default_rng(0)
    nb, T, GH, H, L, n_lv = 2, 19, 8, 3, 5, 5
    A, B = rng.normal(size=(nb, T, GH)), rng.normal(size=(nb, T, GH))
    Ws = [rng.normal(size=(L, H, GH)) for _ in range(3)]
    bs = [rng.normal(size=(L, H)) for _ in range(3)]
    mask = (rng.random((nb, T, L)) > 0.3).astype(np.float64) if with_mask else None
    got = om.gate_preacts(A, B, *Ws, *bs, n_lv, mask)
    for x in range(3):
        ref = _numpy_preacts(A, B, Ws[x], bs[x], n_lv, mask)
        assert np.allclose(got[x], ref, rtol=1e-12, atol=1e-12)
    # plant: a lag off by one must be caught by this comparison
    wrong = _numpy_preacts(A, np.roll(B, 1, axis=1), Ws[0], bs[0], n_lv, mask)
    assert not np.allclose(got[0], wrong, rtol=1e-6, atol=1e-6)
    # plant: W transposed within a level (H == GH would hide it, so shapes differ here)
    with pytest.raises(ValueError):
        _numpy_preacts(A, B, np.swapaxes(Ws[0], 1, 2), bs[0], n_lv, mask)


def test_gate_preacts_zero_source_is_relu_squared():
    rng = np.random.default_rng(1)
    nb, T, GH, H, L = 1, 9, 6, 2, 4
    A = rng.normal(size=(nb, T, GH))
    W = rng.normal(size=(L, H, GH))
    b = rng.normal(size=(L, H))
    got = om.gate_preacts(A, np.zeros_like(A), W, W, W, b, b, b, L)[0]
    for l in range(L):
        assert np.allclose(got[:, :, l], (np.maximum(A, 0) ** 2) @ W[l].T + b[l], atol=1e-12)


# --------------------------------------------------------------------------------------------
# level scan: saturated-gate closed forms (sigmoid(+800) == 1 and sigmoid(-800) == 0 in float64)
# --------------------------------------------------------------------------------------------
def _sat(shape, on):
    return np.full(shape, 800.0 if on else -800.0)


def test_level_scan_window_and_prefix_sums():
    rng = np.random.default_rng(2)
    nb, T, H, hd = 1, 37, 2, 3
    V0 = rng.normal(size=(nb, T, H * hd))
    cs = np.concatenate([np.zeros((nb, 1, H * hd)), np.cumsum(V0, axis=1)], axis=1)
    for n_lv in range(1, 7):
        g = _sat((nb, T, n_lv, H), True)
        V = om.level_scan(g, g, g, V0, H)
        w = 1 << n_lv                                   # window after n_lv levels: 2^n_lv
        t = np.arange(T)
        lo = np.maximum(t - w + 1, 0)
        ref = cs[:, t + 1] - cs[:, lo]
        assert np.allclose(V, ref, atol=1e-9)
    # T <= 2^n_lv: full causal prefix sum
    g = _sat((nb, T, 6, H), True)
    assert np.allclose(om.level_scan(g, g, g, V0, H), cs[:, 1:], atol=1e-9)


def test_level_scan_pure_shift():
    rng = np.random.default_rng(3)
    nb, T, H, hd = 2, 21, 1, 4
    V0 = rng.normal(size=(nb, T, H * hd))
    for n_lv in range(1, 6):
        on = _sat((nb, T, n_lv, H), True)
        V = om.level_scan(on, _sat((nb, T, n_lv, H), False), on, V0, H)   # f = 0, a = r = 1
        src = np.maximum(np.arange(T) - ((1 << n_lv) - 1), 0)
        assert np.allclose(V, V0[:, src], atol=1e-12)


def test_level_scan_plant_dropped_forget_term():
    """A scan that drops f*V (pure message passing) fails the window-sum closed form."""
    rng = np.random.default_rng(4)
    V0 = rng.normal(size=(1, 16, 2))
    on = _sat((1, 16, 3, 1), True)
    off = _sat((1, 16, 3, 1), False)
    good = om.level_scan(on, on, on, V0, 1)
    dropped = om.level_scan(on, off, on, V0, 1)
    assert not np.allclose(good, dropped)


# --------------------------------------------------------------------------------------------
# decode step: the decoder == parallel identity, ring contents included
# --------------------------------------------------------------------------------------------
@pytest.mark.parametrize("nb,T,GH,H,hd,L", [(1, 40, 8, 2, 3, 6), (2, 33, 6, 3, 2, 5)])
def test_decode_steps_equal_parallel_scan(nb, T, GH, H, hd, L):
    rng = np.random.default_rng(5)
    d = H * hd
    A = rng.normal(size=(nb, T, GH))
    Bs = rng.normal(size=(nb, T, GH))
    V0 = rng.normal(size=(nb, T, d))
    Ws = [rng.normal(size=(L, H, GH)) * 0.5 for _ in range(3)]
    bs = [rng.normal(size=(L, H)) for _ in range(3)]
    # parallel: per-level states (state entering level l = scan over the first l levels)
    pres = om.gate_preacts(A, Bs, *Ws, *bs, L)
    states = [V0] + [om.level_scan(*(p[:, :, :l] for p in pres), V0, H) for l in range(1, L + 1)]
    S = (1 << (L + 1)) - 2
    rg = np.zeros((nb, T, L, H))
    ring = np.full((nb, S, d), np.nan)
    for t in range(T):
        Y = om.decode_step(A[:, t], Bs, *Ws, *bs, t, rg, ring, V0[:, t])
        assert np.allclose(Y, states[L][:, t], atol=1e-10), f"step {t}"
        # rg_hist holds r at the source position, all L levels
        assert np.allclose(rg[:, t], 1 / (1 + np.exp(-pres[2][:, t])), atol=1e-12)
        # every live ring slot holds the parallel state entering its level
        for j in range(L):
            for p in range(max(0, t + 1 - (1 << (j + 1))), t + 1):
                assert np.allclose(ring[:, om.ring_slot(j, p)], states[j][:, p], atol=1e-10)


# --------------------------------------------------------------------------------------------
# golden vectors from the reference's CPU eager paths
# --------------------------------------------------------------------------------------------
def test_release_mixer_matches_reference():
    g = golden("release_mixer")
    cfgd = dict(RELEASE_CONFIG, vocab_size=256, eot_token=255, num_layers=1, attn_layers=())
    gen = torch.Generator().manual_seed(99)
    msd = mixer_state_dict(cfgd, gen, "", "parity")
    assert abs(checksum(msd) - float(g["weights_checksum"])) < 1e-6 * float(g["weights_checksum"])
    T, d, H = 40, 1024, 16
    x = torch.randn(1, T, d, generator=gen).double().numpy()
    W = {k: v.double().numpy() for k, v in msd.items()}
    A = x @ W["gate_hidden.weight"].T
    Bs = x @ W["gate_hidden_src.weight"].T
    V0 = x @ W["linear_in.weight"].T
    n_lv = om.active_levels(12, T)
    Wb = [W[k] for k in ("gate_out", "forget_out", "reset_out", "gate_out_bias", "forget_out_bias",
                         "reset_out_bias")]
    for mask, key in ((g["tree_mask"], "doc"), (None, "level")):
        m = None if mask is None else mask[..., :n_lv]
        pres = om.gate_preacts(A, Bs, *Wb, n_lv, m)
        V = om.level_scan(*pres, V0, H, m)
        y = V @ W["linear_out.weight"].T
        if key == "doc":
            assert rel_err(V, g["V_doc"]) < 2e-5
        assert rel_err(y, g[f"y_{key}"]) < 2e-5


@pytest.mark.parametrize("name", sorted(TINY_CONFIGS))
def test_torch_oracle_matches_reference(name):
    g = golden(name)
    cfgd, sd = tiny(name)
    assert abs(checksum(sd) - float(g["weights_checksum"])) < 1e-6 * float(g["weights_checksum"])
    spec = te.Spec(type("C", (), cfgd))
    logits = te.forward(sd, spec, torch.from_numpy(g["ids"]))
    assert rel_err(logits, g["logits"]) < 1e-5
    dec = te.EagerDecoder(sd, spec)
    pl = dec.prefill(torch.from_numpy(g["prompts"]))
    assert rel_err(pl, g["prefill_logits"]) < 1e-5
    steps = torch.stack([dec.step(torch.from_numpy(g["nexts"][:, j])) for j in range(g["nexts"].shape[1])], 1)
    assert rel_err(steps, g["step_logits"]) < 1e-5
    c0 = dec.caches[0]
    Tn = g["B_hist0"].shape[1]
    assert max_abs(c0["B_hist"][:, :Tn], g["B_hist0"]) < 1e-5
    assert max_abs(c0["rg_hist"][:, :Tn], g["rg_hist0"]) < 1e-5
    assert max_abs(c0["V_ring"], g["V_ring0"]) < 1e-5
    # greedy generation through the eager decoder reproduces the reference's tokens
    prompt = torch.from_numpy(g["gen"][:, :6])
    d2 = te.EagerDecoder(sd, spec)
    toks = [prompt]
    lg = d2.prefill(prompt)[:, -1]
    for _ in range(g["gen"].shape[1] - 6):
        nxt = lg.argmax(-1)
        toks.append(nxt[:, None])
        lg = d2.step(nxt)
    assert np.array_equal(torch.cat(toks, 1).numpy(), g["gen"])


def test_golden_plant_detects_wrong_rope_pairing():
    """The golden logits pin the attention composition: pairing halves instead of interleaved
    elements (a plausible RoPE mistake) moves the logits far beyond the tolerance."""
    g = golden("tiny_a")
    cfgd, sd = tiny("tiny_a")
    spec = te.Spec(type("C", (), cfgd))
    orig = te.rope

    def halves(x, cos, sin):
        h = x.shape[-1] // 2
        x1, x2 = x[..., :h], x[..., h:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)

    te.rope = halves
    try:
        bad = te.forward(sd, spec, torch.from_numpy(g["ids"]))
    finally:
        te.rope = orig
    assert rel_err(bad, g["logits"]) > 1e-3
