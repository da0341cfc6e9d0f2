"""Host-side contracts of the product package on the CPU (no GPU needed).

The product's eager mode and eager decoder are the reference's public API; they are checked against
the reference's own golden vectors, and the reference tests' invariants are re-run on seeded
weights (reference tests/test_parity.py:30-64, tests/test_decoding.py:47-203). Error contracts
mirror the reference's exceptions.
"""

import numpy as np
import pytest
import torch

from helpers import golden, max_abs, product_model, rel_err, tiny
from weights import TINY_CONFIGS


@pytest.fixture(scope="module", params=sorted(TINY_CONFIGS))
def tiny_model(request):
    cfgd, sd = tiny(request.param)
    return request.param, cfgd, product_model(cfgd, sd)


def test_forward_matches_reference_golden(tiny_model):
    name, cfgd, m = tiny_model
    g = golden(name)
    with torch.no_grad():
        logits = m(torch.from_numpy(g["ids"])).logits
    assert rel_err(logits, g["logits"]) < 1e-5


def test_incremental_decoder_matches_reference_golden(tiny_model):
    from dispatcher_hybrid.decoding import IncrementalDecoder
    name, cfgd, m = tiny_model
    g = golden(name)
    dec = IncrementalDecoder(m)
    pl = dec.prefill(torch.from_numpy(g["prompts"]))
    assert rel_err(pl, g["prefill_logits"]) < 1e-5
    st = torch.stack([dec.step(torch.from_numpy(g["nexts"][:, j])) for j in range(8)], 1)
    assert rel_err(st, g["step_logits"]) < 1e-5
    c0 = dec.caches[0]
    Tn = g["B_hist0"].shape[1]
    assert max_abs(c0.B_hist[:, :Tn], g["B_hist0"]) < 1e-5
    assert max_abs(c0.rg_hist[:, :Tn], g["rg_hist0"]) < 1e-5
    assert max_abs(c0.V_ring, g["V_ring0"]) < 1e-5


def test_fast_generate_eager_matches_reference_golden(tiny_model):
    name, cfgd, m = tiny_model
    g = golden(name)
    out = m.fast_generate(torch.from_numpy(g["gen"][:, :6]), max_new_tokens=g["gen"].shape[1] - 6,
                          decoder="eager")
    assert np.array_equal(out.numpy(), g["gen"])


def test_generate_matches_fast_generate(tiny_model):
    """reference tests/test_decoding.py:89-95 and tests/test_parity.py:61-64: HF generate() on the
    product model runs (shape) and gives greedy fast_generate's tokens; both equal the reference's
    own greedy tokens (golden)."""
    name, cfgd, m = tiny_model
    g = golden(name)
    ids = torch.from_numpy(g["gen"][:, :6])
    n = g["gen"].shape[1] - 6
    a = m.generate(ids, max_new_tokens=n, do_sample=False)
    assert a.shape == (ids.shape[0], 6 + n)
    assert torch.equal(a, m.fast_generate(ids, max_new_tokens=n, decoder="eager"))
    assert np.array_equal(a.numpy(), g["gen"])


def test_decoder_matches_parallel_forward(tiny_model):
    """reference tests/test_decoding.py:33-47: prefill 48, 12 steps, logits == parallel forward."""
    from dispatcher_hybrid.decoding import IncrementalDecoder
    _, cfgd, m = tiny_model
    torch.manual_seed(0)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (60,))
    with torch.no_grad():
        ref = m(ids.unsqueeze(0)).logits[0, 48:]
    dec = IncrementalDecoder(m)
    dec.prefill(ids[:48])
    got = torch.stack([dec.step(ids[t]) for t in range(48, 60)])
    assert (got.argmax(-1) == ref.argmax(-1)).all()
    assert (got - ref).abs().max().item() < 1e-4


def test_causality_exact():
    """reference tests/test_parity.py:30-41: a token never changes earlier logits."""
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd)
    torch.manual_seed(0)
    ids = torch.randint(0, 250, (1, 64))
    with torch.no_grad():
        base = m(ids).logits
        for cut in (5, 17, 40, 63):
            poked = ids.clone()
            poked[0, cut] = (poked[0, cut] + 97) % 250
            after = m(poked).logits
            assert (after[0, :cut] - base[0, :cut]).abs().max().item() == 0.0


def test_doc_reset_bounds_cross_document_influence():
    """reference tests/test_parity.py:44-58: only attention crosses an EOT."""
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd)
    eot = cfgd["eot_token"]
    torch.manual_seed(1)
    tail = torch.randint(0, 250, (1, 20))
    a = torch.cat([torch.randint(0, 250, (1, 20)), torch.tensor([[eot]]), tail], 1)
    b = torch.cat([torch.randint(0, 250, (1, 20)), torch.tensor([[eot]]), tail], 1)
    with torch.no_grad():
        da = (m(a).logits[0, 21:] - m(b).logits[0, 21:]).abs().max().item()
    assert da < 20.0
    # with attention removed the tree alone must isolate the documents exactly
    cfg2 = dict(cfgd, attn_layers=())
    sd2 = {k: v for k, v in sd.items()}
    from weights import make_state_dict
    sd2 = make_state_dict(cfg2, 5)
    m2 = product_model(cfg2, sd2)
    with torch.no_grad():
        assert (m2(a).logits[0, 21:] - m2(b).logits[0, 21:]).abs().max().item() == 0.0


def test_doc_reset_mask_one_gather_equals_per_level_form():
    """The doc-reset mask built with one gather of the cached (T, L) source-index table equals the
    per-level form of reference modeling_dispatcher.py:311-323 (doc ids compared at (t - 2^l) mod T,
    level by level), bit for bit, over lengths around the level horizons and EOT patterns."""
    for name in sorted(TINY_CONFIGS):
        cfgd, sd = tiny(name)
        m = product_model(cfgd, sd)
        if not m.config.doc_reset:
            continue
        g = torch.Generator().manual_seed(3)
        for T in (1, 2, 5, 37, 64):
            ids = torch.randint(0, cfgd["vocab_size"], (3, T), generator=g)
            ids[0, T // 2] = m.config.eot_token
            ids[2, ::3] = m.config.eot_token
            got = m._tree_mask(ids, T)
            mask = m.level_mask(T, ids.device, m.embedding.weight.dtype)
            is_eot = (ids == m.config.eot_token).to(mask.dtype)
            doc = torch.cumsum(is_eot, dim=1) - is_eot
            t = torch.arange(T)
            same = torch.stack([doc == doc[:, (t - (1 << l)) % T] for l in range(m.config.levels)], dim=-1)
            ref = mask.unsqueeze(0) * same.to(mask.dtype)[..., :mask.shape[-1]]
            assert torch.equal(got, ref), (name, T)


def test_batched_matches_single():
    """reference tests/test_decoding.py:134-153."""
    from dispatcher_hybrid.decoding import IncrementalDecoder
    cfgd, sd = tiny("tiny_b")
    m = product_model(cfgd, sd)
    torch.manual_seed(0)
    prompts = torch.randint(0, 250, (3, 20))
    nexts = torch.randint(0, 250, (3, 8))
    dec = IncrementalDecoder(m)
    batched = [dec.prefill(prompts)[:, -1]] + [dec.step(nexts[:, j]) for j in range(8)]
    batched = torch.stack(batched, 1)
    for b in range(3):
        d1 = IncrementalDecoder(m)
        solo = torch.stack([d1.prefill(prompts[b])[-1]] + [d1.step(nexts[b, j]) for j in range(8)])
        assert (batched[b] - solo).abs().max().item() < 1e-4


def test_ring_cache_layout():
    """reference tests/test_decoding.py:121-131: ring, not dense."""
    from dispatcher_hybrid.decoding import IncrementalDecoder
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd)
    dec = IncrementalDecoder(m)
    dec.prefill(torch.randint(0, 250, (12,)))
    tree = next(c for c in dec.caches if hasattr(c, "V_ring"))
    assert tree.V_ring.shape[1] == 2 ** (tree.L + 1) - 2
    assert [int(o) for o in tree.offsets] == [2 ** (j + 1) - 2 for j in range(tree.L)]
    assert [int(k) for k in tree.masks] == [2 ** (j + 1) - 1 for j in range(tree.L)]
    assert (tree.L + 1) * cfgd["max_len"] / tree.V_ring.shape[1] > 3


def test_fast_generate_api_contracts():
    """reference tests/test_decoding.py:181-203."""
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd)
    torch.manual_seed(0)
    ids = torch.tensor([[10, 11, 12, 13]])
    out = m.fast_generate(ids, max_new_tokens=6, do_sample=True, temperature=1.0,
                          num_return_sequences=3, decoder="eager")
    assert out.shape == (3, 10) and (out[:, :4] == ids).all()
    ids2 = torch.randint(0, 250, (2, 8))
    eos = int(m.fast_generate(ids2[:1], max_new_tokens=1, decoder="eager")[0, -1])
    out = m.fast_generate(ids2, max_new_tokens=6, decoder="eager", eos_token_id=eos)
    assert int(out[0, 8]) == eos and (out[0, 8:] == eos).all()
    assert out.shape[0] == 2 and out.shape[1] <= 14
    # context cap: fast_generate stops at max_len
    full = torch.randint(0, 250, (1, cfgd["max_len"] - 2))
    out = m.fast_generate(full, max_new_tokens=10, decoder="eager")
    assert out.shape[1] == cfgd["max_len"] + 1


def test_error_contracts():
    from dispatcher_hybrid import DispatcherConfig
    from dispatcher_hybrid.decoding import GraphedHybridDecoder, IncrementalDecoder
    with pytest.raises(ValueError, match="power of two"):
        DispatcherConfig(max_len=1000)
    with pytest.raises(ValueError, match="divisible"):
        DispatcherConfig(d_model=100, num_heads=16)
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd)
    with pytest.raises(ValueError, match="requires input_ids"):
        m(None)
    with pytest.raises(ValueError, match="exceeds max_len"):
        m(torch.zeros(1, cfgd["max_len"] + 1, dtype=torch.long))
    with pytest.raises(ValueError, match="single prompt"):
        m.fast_generate(torch.zeros(2, 3, dtype=torch.long), do_sample=True, num_return_sequences=2)
    with pytest.raises(ValueError, match="identical rows"):
        m.fast_generate(torch.zeros(1, 3, dtype=torch.long), num_return_sequences=2)
    with pytest.raises(ValueError, match="decoder dtype"):
        IncrementalDecoder(m, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="document separator"):
        IncrementalDecoder(m).prefill(torch.tensor([1, 2, cfgd["eot_token"], 3]))
    dec = IncrementalDecoder(m)
    with pytest.raises(ValueError, match="exceeds max_len"):
        dec.prefill(torch.zeros(cfgd["max_len"] + 1, dtype=torch.long))
    dec.prefill(torch.zeros(2, cfgd["max_len"] - 1, dtype=torch.long))
    with pytest.raises(ValueError, match="tokens for batch"):
        dec.step(torch.zeros(3, dtype=torch.long))
    dec.step(torch.zeros(2, dtype=torch.long))
    with pytest.raises(ValueError, match="context exhausted"):
        dec.step(torch.zeros(2, dtype=torch.long))
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="requires a GPU"):
            GraphedHybridDecoder(m)


def test_fused_gates_switch_and_cpu_refusal():
    """enable_fused_gates toggles every mixer; on CPU tensors the fused path raises instead of
    silently running eager."""
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd)
    ids = torch.randint(0, 250, (1, 16))
    with torch.no_grad():
        before = m(ids).logits
    assert m.enable_fused_gates() is m
    assert all(b.mixer.use_fused_gates for b in m.blocks if hasattr(b, "mixer"))
    with pytest.raises(RuntimeError, match="on the CPU"):
        with torch.no_grad():
            m(ids)
    m.enable_fused_gates(False)
    assert not any(b.mixer.use_fused_gates for b in m.blocks if hasattr(b, "mixer"))
    with torch.no_grad():
        assert torch.equal(m(ids).logits, before)


def test_fused_wrappers_refuse_cpu_tensors():
    """The HIP wrappers have no CPU implementation: CPU tensors raise before any library call, and
    the module-level routing helpers report that the fused GEMMs do not apply to them."""
    from dispatcher_hybrid import fused_gates as fg
    x = torch.randn(4, 64, dtype=torch.bfloat16)
    w = torch.randn(8, 64, dtype=torch.bfloat16)
    ids = torch.zeros(2, 16, dtype=torch.int64)
    for call in (lambda: fg.fused_swiglu(x, w, w), lambda: fg.fused_projections(x, [w]),
                 lambda: fg.silu_mul(x, x), lambda: fg.tree_mask(ids, 4, 7, torch.bfloat16)):
        with pytest.raises(RuntimeError, match="must be on the GPU"):
            call()
    lin = torch.nn.Linear(64, 8, bias=False).to(torch.bfloat16)
    assert not fg.swiglu_fits(x, lin, lin)
    assert not fg.projections_fit(x, [lin])
    # on the CPU the routing helper is the library call itself
    assert torch.equal(fg.project(x, [lin], fg.OUT_GEMM_MAX_ROWS)[0], lin(x))


def test_reference_init_scheme():
    """The product's own init: N(0, 0.02), W1s zero, biases -2/+2/+2, tied head."""
    from dispatcher_hybrid import DispatcherHybridForCausalLM
    from helpers import config
    torch.manual_seed(0)
    m = DispatcherHybridForCausalLM(config(TINY_CONFIGS["tiny_a"]))
    mx = m.blocks[0].mixer
    assert torch.count_nonzero(mx.gate_hidden_src.weight) == 0
    assert abs(mx.gate_out.std().item() - 0.02) < 0.005
    assert torch.all(mx.gate_out_bias == -2.0) and torch.all(mx.forget_out_bias == 2.0)
    assert torch.all(mx.reset_out_bias == 2.0)
    assert m.lm_head.weight.data_ptr() == m.embedding.weight.data_ptr()
