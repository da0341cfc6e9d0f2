"""dh_decode_persistent_step (one cooperative launch per batch-1 bf16 greedy step) against the
graph of launches it replaces (FusedGraphedHybridDecoder.step_greedy with persistent=False,
reference dispatcher_hybrid/decoding.py:437-488): the same arithmetic, so the logits after every
step, the picked tokens and every decode-state buffer must be equal bit for bit."""

import pytest
import torch

from helpers import product_model, tiny
from weights import make_state_dict

pytestmark = pytest.mark.gpu
DEV = "cuda"

# head width 64, two attention layers (window 128 < the decoded context), 9 levels
MID = dict(vocab_size=2048, d_model=512, num_heads=8, dim_feedforward=1024, num_layers=4, max_len=512,
           attn_layers=(2, 4), attn_window=128, doc_reset=True, eot_token=2047)


def _pair(m, prompt):
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    dp, dg = FusedGraphedHybridDecoder(m), FusedGraphedHybridDecoder(m, persistent=False)
    for dec in (dp, dg):
        dec.greedy_start(dec.prefill(prompt)[:, -1])
    return dp, dg


def _state(dec):
    out = []
    for c in dec.inner.caches:
        out += [c.B_hist, c.rg_hist, c.V_ring] if hasattr(c, "V_ring") else [c.k, c.v]
    return out


def _run_and_compare(dp, dg, steps):
    for i in range(steps):
        dp.step_greedy()
        dg.step_greedy()
        assert torch.equal(dp.logits_out, dg.logits_out), f"logits differ at step {i}"
        assert torch.equal(dp.token_buf, dg.token_buf), f"token differs at step {i}"
    assert dp._pers, "the one-launch step must have been used"
    assert dp.persistent_status() == (0, 0)
    assert torch.equal(dp.t_buf, dg.t_buf) and dp.t == dg.t
    assert torch.equal(dp.tok_hist, dg.tok_hist)
    for j, (a, b) in enumerate(zip(_state(dp), _state(dg))):
        assert torch.equal(a, b), f"decode state buffer {j} differs"


def test_persistent_mid_model_bit_exact_and_rerun():
    """A 4-layer bf16 model (two attention layers, window 128): 160 steps from a 20-token prompt
    (the window slides), then the same decoder prefilled again with another prompt decodes the
    same positions once more (words left by the first run carry stale tags)."""
    sd = make_state_dict(MID, 7)
    m = product_model(MID, sd, device=DEV, dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(3)
    prompt = torch.randint(0, 2047, (1, 20), device=DEV, generator=g)
    print("persistent: mid model, 160 steps", flush=True)
    dp, dg = _pair(m, prompt)
    _run_and_compare(dp, dg, 160)
    print("persistent: mid model, rerun over the same positions", flush=True)
    prompt2 = torch.randint(0, 2047, (1, 20), device=DEV, generator=g)
    for dec in (dp, dg):
        dec.greedy_start(dec.prefill(prompt2)[:, -1])
    _run_and_compare(dp, dg, 40)


def test_persistent_release_model_bit_exact():
    """The released 292M architecture (random init), a 1100-token prompt (attention window 1024
    full and sliding), 24 steps."""
    from dispatcher_hybrid import DispatcherConfig, DispatcherHybridForCausalLM
    torch.manual_seed(0)
    with torch.device(DEV):
        m = DispatcherHybridForCausalLM(DispatcherConfig())
    m = m.to(torch.bfloat16).eval()
    prompt = torch.randint(0, 50256, (1, 1100), device=DEV, generator=torch.Generator(device=DEV).manual_seed(5))
    print("persistent: release model, 24 steps", flush=True)
    dp, dg = _pair(m, prompt)
    _run_and_compare(dp, dg, 24)


def test_persistent_not_used_where_unsupported():
    """fp32 models, batch > 1 and widths outside the kernel keep the graph of launches."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16)     # d = 128: not supported
    dec = FusedGraphedHybridDecoder(m)
    dec.greedy_start(dec.prefill(torch.randint(0, 250, (1, 8), device=DEV))[:, -1])
    dec.step_greedy()
    assert dec._pers is False
    mf = product_model(MID, make_state_dict(MID, 7), device=DEV)     # fp32
    dec = FusedGraphedHybridDecoder(mf)
    dec.greedy_start(dec.prefill(torch.randint(0, 2047, (1, 8), device=DEV))[:, -1])
    dec.step_greedy()
    assert dec._pers is False


def test_persistent_every_position_from_one_token_to_max_len():
    """A 1-token prompt decoded to the end of the context (t = 1 .. max_len - 1): every level's first
    source, the attention window filling and sliding (window 64 of 256), the last position; then
    the decoder refuses a step past max_len as the graph path does."""
    cfg = dict(MID, max_len=256, attn_window=64)
    m = product_model(cfg, make_state_dict(cfg, 11), device=DEV, dtype=torch.bfloat16)
    prompt = torch.randint(0, 2047, (1, 1), device=DEV, generator=torch.Generator(device=DEV).manual_seed(9))
    print("persistent: positions 1..255", flush=True)
    dp, dg = _pair(m, prompt)
    _run_and_compare(dp, dg, 255)
    assert dp.t == 256
    with pytest.raises(ValueError, match="context exhausted"):
        dp.step_greedy()


def test_fast_generate_greedy_uses_one_launch_step():
    """fast_generate's greedy branch (no eos) through the fused decoder gives the same tokens with
    the one-launch step as with the graph of launches."""
    from dispatcher_hybrid import decoding
    m = product_model(MID, make_state_dict(MID, 7), device=DEV, dtype=torch.bfloat16)
    prompt = torch.randint(0, 2047, (1, 30), device=DEV, generator=torch.Generator(device=DEV).manual_seed(4))
    out = m.fast_generate(prompt, max_new_tokens=40, decoder="fused")
    orig = decoding.FusedGraphedHybridDecoder.__init__.__defaults__
    decoding.FusedGraphedHybridDecoder.__init__.__defaults__ = (None, None, False)   # persistent=False
    try:
        ref = m.fast_generate(prompt, max_new_tokens=40, decoder="fused")
    finally:
        decoding.FusedGraphedHybridDecoder.__init__.__defaults__ = orig
    assert torch.equal(out, ref)


def test_persistent_reprefill_at_other_batch_sizes():
    """Prefilling the same decoder again at another batch size reallocates its caches: the one-launch
    step's layer table (raw cache addresses) is derived again, so batch 2 runs the graph of launches
    and batch 1 again the one-launch step, each equal to a decoder that never used it."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    m = product_model(MID, make_state_dict(MID, 7), device=DEV, dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(12)
    p1 = torch.randint(0, 2047, (1, 20), device=DEV, generator=g)
    p2 = torch.randint(0, 2047, (2, 24), device=DEV, generator=g)
    dp, dg = FusedGraphedHybridDecoder(m), FusedGraphedHybridDecoder(m, persistent=False)
    print("persistent: batch 1 -> 2 -> 1", flush=True)
    for prompt, steps, one_launch in ((p1, 6, True), (p2, 6, False), (p1, 8, True)):
        for dec in (dp, dg):
            dec.greedy_start(dec.prefill(prompt)[:, -1])
        for i in range(steps):
            dp.step_greedy()
            dg.step_greedy()
            assert torch.equal(dp.logits_out, dg.logits_out), f"logits differ at step {i}, batch {prompt.shape[0]}"
            assert torch.equal(dp.token_buf, dg.token_buf)
        assert bool(dp._pers) == one_launch
        for j, (a, b) in enumerate(zip(_state(dp), _state(dg))):
            assert torch.equal(a, b), f"decode state buffer {j} differs (batch {prompt.shape[0]})"


def test_persistent_status_set_redoes_steps_on_graph_path():
    """Recovery after a one-launch step reports a timed-out wait, forced from the host: the status
    word of the decoder's scratch is set before three steps, so none of them advances the device
    position or writes a token (every workgroup still exits normally). check_persistent() then
    redoes the three steps from the device position through the graph of launches, which the decoder
    keeps using; tokens, logits and every state buffer equal those of a decoder that ran the graph of
    launches throughout."""
    m = product_model(MID, make_state_dict(MID, 7), device=DEV, dtype=torch.bfloat16)
    prompt = torch.randint(0, 2047, (1, 30), device=DEV, generator=torch.Generator(device=DEV).manual_seed(8))
    dp, dg = _pair(m, prompt)
    dp.persistent_check_every = 0
    _run_and_compare(dp, dg, 5)
    t0 = dp.t
    status = dp._pers["scratch"][8:16].view(torch.int32)
    status.copy_(torch.tensor([1, 2001], dtype=torch.int32))   # abort flag; phase 0, "time"
    print("persistent: three steps with the status word set", flush=True)
    for _ in range(3):
        dp.step_greedy()
    assert dp.t == t0 + 3 and int(dp.t_buf.item()) == t0, "an aborted step advanced the device position"
    with pytest.warns(RuntimeWarning, match="timed out"):
        assert dp.check_persistent() == 3
    assert dp._pers is False and not dp.use_persistent and dp.t == t0 + 3
    for _ in range(3):
        dg.step_greedy()
    assert torch.equal(dp.logits_out, dg.logits_out) and torch.equal(dp.token_buf, dg.token_buf)
    for i in range(6):
        dp.step_greedy()
        dg.step_greedy()
        assert torch.equal(dp.logits_out, dg.logits_out), f"logits differ at step {i} after recovery"
    assert torch.equal(dp.t_buf, dg.t_buf) and dp.t == dg.t and torch.equal(dp.tok_hist, dg.tok_hist)
    for j, (a, b) in enumerate(zip(_state(dp), _state(dg))):
        assert torch.equal(a, b), f"decode state buffer {j} differs"
