"""Model-level parity of the fused HIP paths (enable_fused_gates, FusedGraphedHybridDecoder,
fast_generate(decoder="fused")) against the oracle, the reference's golden vectors and the reference
tests' contracts (reference tests/test_decoding.py:33-178)."""

import numpy as np
import pytest
import torch

from helpers import (argmax_agree, bf16_vs_truth, decisive_argmax_agree, golden, max_abs, preact_bound, product_model,
                     rel_err, tiny)
from dispatcher_hybrid.numerics import fp32_product_accumulation
from oracle import torch_eager as te
from weights import RELEASE_CONFIG, TINY_CONFIGS, make_state_dict

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", params=sorted(TINY_CONFIGS))
def tiny_gpu(request):
    cfgd, sd = tiny(request.param)
    return request.param, cfgd, sd, product_model(cfgd, sd, device=DEV)


def test_fused_forward_fp32_matches_reference(tiny_gpu):
    """enable_fused_gates() in fp32 (doc-reset masks active) vs the reference's logits."""
    name, cfgd, sd, m = tiny_gpu
    g = golden(name)
    ids = torch.from_numpy(g["ids"]).to(DEV)
    m.enable_fused_gates()
    try:
        with torch.no_grad():
            got = m(ids).logits
    finally:
        m.enable_fused_gates(False)
    assert rel_err(got.cpu(), g["logits"]) < 1e-4


def test_fused_forward_bf16_tracks_eager(tiny_gpu):
    """reference tests/test_decoding.py:108-118: fused bf16 prefill argmax agreement > 0.95."""
    name, cfgd, sd, m = tiny_gpu
    mb = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16)
    torch.manual_seed(0)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (2, 64), device=DEV)
    with torch.no_grad():
        eager = mb(ids).logits.float()
        mb.enable_fused_gates()
        fused = mb(ids).logits.float()
    ref = te.forward(sd, te.Spec(type("C", (), cfgd)), ids.cpu())
    assert argmax_agree(fused.cpu(), ref) > 0.95
    assert argmax_agree(fused, eager) > 0.95


def test_fused_tree_mask_equals_eager_tree_mask():
    """With enable_fused_gates() the doc-reset tree mask comes from dh_tree_mask: the same values,
    shape and dtype as the torch formula the eager forward uses."""
    for name in sorted(TINY_CONFIGS):
        cfgd, sd = tiny(name)
        for dtype in (torch.float32, torch.bfloat16):
            m = product_model(cfgd, sd, device=DEV, dtype=dtype)
            if not m.config.doc_reset:
                continue
            g = torch.Generator().manual_seed(5)
            for T in (1, 3, 64, 200):
                ids = torch.randint(0, cfgd["vocab_size"], (3, T), generator=g)
                ids[0, T // 2] = m.config.eot_token
                ids[2, ::3] = m.config.eot_token
                ids = ids.to(DEV)
                ref = m._tree_mask(ids, T)
                got = m.enable_fused_gates()._tree_mask(ids, T)
                m.enable_fused_gates(False)
                assert got.dtype == ref.dtype and torch.equal(got, ref), (name, dtype, T)


def test_fused_forward_sees_in_place_bias_updates(tiny_gpu):
    """The fused path reads bf16 gate biases through cached fp32 copies: an in-place update of a
    bias must reach the next fused forward (the copy follows the tensor's version counter)."""
    name, cfgd, sd, m = tiny_gpu
    mb = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16).enable_fused_gates()
    torch.manual_seed(1)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (1, 48), device=DEV)
    with torch.no_grad():
        before = mb(ids).logits.clone()
        for blk in mb.blocks:
            if hasattr(blk, "mixer"):
                blk.mixer.reset_out_bias.add_(-3.0)
                blk.mixer.gate_out_bias.add_(1.5)
        after = mb(ids).logits
        mb.enable_fused_gates(False)
        eager = mb(ids).logits
    assert not torch.equal(before, after)
    assert argmax_agree(after.float(), eager.float()) > 0.95


def test_fused_autograd_matches_eager():
    """Gradients through dispatcher::gate_preacts_fwd/bwd equal the eager mixer's (fp32)."""
    cfgd, sd = tiny("tiny_a")
    m_e = product_model(cfgd, sd, device=DEV).train()
    m_f = product_model(cfgd, sd, device=DEV).train().enable_fused_gates()
    g = golden("tiny_a")
    ids = torch.from_numpy(g["ids"]).to(DEV)
    labels = ids.clone()
    loss_e = m_e(ids, labels=labels).loss
    loss_f = m_f(ids, labels=labels).loss
    loss_e.backward()
    loss_f.backward()
    assert abs(loss_e.item() - loss_f.item()) < 1e-5 * abs(loss_e.item())
    for (n, pe), (_, pf) in zip(m_e.named_parameters(), m_f.named_parameters()):
        assert rel_err(pf.grad, pe.grad) < 1e-3, n


def _gate_eager(A, Bs, params, n_lv, m3):
    """The reference's gate pre-activations (modeling_dispatcher.py:100-109) in the inputs' dtype."""
    from dispatcher_hybrid.modeling_dispatcher import level_gate_matmul
    lagged = torch.stack([torch.roll(Bs, shifts=1 << l, dims=1) for l in range(n_lv)], dim=2)
    hidden = torch.relu(A.unsqueeze(2) + lagged * m3.unsqueeze(-1).to(A.dtype)) ** 2
    return [level_gate_matmul(hidden, W[:n_lv]) + b[:n_lv] for W, b in params]


def test_fused_gate_backward_bf16_release_widths():
    """bf16 gradients of dispatcher::gate_preacts_fwd (its bwd op, reference fused_gates.py:225-257)
    at the released widths (GH 1024, 16 heads, 12 levels; b 2, T 512, a doc-reset style mask) for
    dA, dB and the three readout weights and biases: each within 1.25x the eager bf16 autograd's
    relative error against float32 autograd of the same formula (or 2e-3)."""
    torch.manual_seed(11)
    b, T, GH, H, L = 2, 512, 1024, 16, 12
    A = (torch.randn(b, T, GH, device=DEV) * 0.5).bfloat16()
    Bs = (torch.randn(b, T, GH, device=DEV) * 0.5).bfloat16()
    params = [((torch.randn(L, H, GH, device=DEV) / 32).bfloat16(), (torch.randn(L, H, device=DEV) * 0.1).bfloat16())
              for _ in range(3)]
    t = torch.arange(T, device=DEV)
    m3 = (t[None, :, None] >= (1 << torch.arange(L, device=DEV))[None, None, :]).float().expand(b, T, L).clone()
    m3[0, 200:, 3:] = 0                                   # a document boundary in row 0
    m3[1, 37, :] = 0
    G = [torch.randn(b, T, L, H, device=DEV) for _ in range(3)]

    def grads(fn, dtype, dev=DEV):
        leaf = lambda x: x.detach().to(dev, dtype).clone().requires_grad_()
        leaves = [leaf(A), leaf(Bs)]
        ps = [(leaf(W), leaf(bb)) for W, bb in params]
        outs = fn(leaves[0], leaves[1], ps, m3.to(dev))
        loss = sum((o.float() * g.to(dev)).sum() for o, g in zip(outs, G))
        loss.backward()
        return [x.to(DEV) for x in [leaves[0].grad, leaves[1].grad] + [x.grad for W, bb in ps for x in (W, bb)]]

    fused = grads(lambda a, bs, ps, mk: torch.ops.dispatcher.gate_preacts_fwd(
        a, bs, ps[0][0], ps[1][0], ps[2][0], ps[0][1], ps[1][1], ps[2][1], L, mk), torch.bfloat16)
    # eager bf16 autograd on the CPU: its bmm backward takes transposed bf16 operands, kept off the GPU
    eager = grads(lambda a, bs, ps, mk: _gate_eager(a, bs, ps, L, mk), torch.bfloat16, "cpu")
    truth = grads(lambda a, bs, ps, mk: _gate_eager(a, bs, ps, L, mk), torch.float32)
    names = ["dA", "dB", "dWi", "dbi", "dWf", "dbf", "dWr", "dbr"]
    for n, f, e, tr in zip(names, fused, eager, truth):
        assert f.dtype == torch.bfloat16 and f.shape == tr.shape, n
        ef, ee = rel_err(f.float(), tr), rel_err(e.float(), tr)
        print(f"gate bwd bf16 {n}: fused rel {ef:.2e}  eager bf16 rel {ee:.2e}", flush=True)
        assert ef <= max(1.25 * ee, 2e-3), n


def _compare_decoder(dec_cls, m, vocab, device, prompt=40, steps=12, tol=1e-4):
    """reference tests/test_decoding.py:33-44 on seeded weights."""
    torch.manual_seed(0)
    ids = torch.randint(0, vocab - 1, (prompt + steps,), device=device)
    with torch.no_grad():
        ref = m(ids.unsqueeze(0)).logits[0, prompt:].float()
    dec = dec_cls(m)
    dec.prefill(ids[:prompt])
    got = torch.stack([dec.step(ids[t]).float() for t in range(prompt, prompt + steps)])
    assert (got.argmax(-1) == ref.argmax(-1)).all(), "argmax disagrees with the parallel forward"
    gap = (got - ref).abs().max().item()
    assert gap < tol, f"{dec_cls.__name__}: max|dlogit| {gap:.3e}"


def test_graphed_decoder_matches_parallel_forward(tiny_gpu):
    from dispatcher_hybrid.decoding import GraphedHybridDecoder
    name, cfgd, sd, m = tiny_gpu
    _compare_decoder(GraphedHybridDecoder, m, cfgd["vocab_size"], DEV)


def test_fused_decoder_matches_parallel_forward(tiny_gpu):
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    name, cfgd, sd, m = tiny_gpu
    _compare_decoder(FusedGraphedHybridDecoder, m, cfgd["vocab_size"], DEV)


def test_fused_decoder_matches_reference_golden(tiny_gpu):
    """Fused decoder logits and layer-0 state vs the reference's eager decoder (fp32)."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    name, cfgd, sd, m = tiny_gpu
    g = golden(name)
    dec = FusedGraphedHybridDecoder(m)
    pl = dec.prefill(torch.from_numpy(g["prompts"]).to(DEV))
    assert rel_err(pl.cpu(), g["prefill_logits"]) < 1e-4
    st = torch.stack([dec.step(torch.from_numpy(g["nexts"][:, j]).to(DEV)) for j in range(8)], 1)
    assert rel_err(st.cpu(), g["step_logits"]) < 1e-4
    c0 = dec.inner.caches[0]
    Tn = g["B_hist0"].shape[1]
    assert max_abs(c0.B_hist[:, :Tn].cpu(), g["B_hist0"]) < 1e-4
    assert max_abs(c0.rg_hist[:, :Tn].cpu(), g["rg_hist0"]) < 1e-4
    assert max_abs(c0.V_ring.cpu(), g["V_ring0"]) < 1e-4


def test_fused_decoder_state_equals_eager_decoder_state():
    """Ring slots, rg_hist and B_hist written by the fused step match the eager step's."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    cfgd, sd = tiny("tiny_b")
    m = product_model(cfgd, sd, device=DEV)
    torch.manual_seed(3)
    prompts = torch.randint(0, 250, (3, 9), device=DEV)
    nexts = torch.randint(0, 250, (3, 20), device=DEV)
    decs = [IncrementalDecoder(m), FusedGraphedHybridDecoder(m)]
    for d in decs:
        d.prefill(prompts)
        for j in range(nexts.shape[1]):
            d.step(nexts[:, j])
    for ce, cf in zip(decs[0].caches, decs[1].inner.caches):
        if hasattr(ce, "V_ring"):
            assert max_abs(cf.V_ring, ce.V_ring) < 1e-5
            assert max_abs(cf.rg_hist, ce.rg_hist) < 1e-5
            assert max_abs(cf.B_hist, ce.B_hist) < 1e-5


@pytest.mark.parametrize("T", [1, 2, 3, 5, 17, 40, 63])
def test_fused_prefill_state_equals_eager_prefill(T):
    """The fused decoder's prefill (parallel gate kernels + the scan's ring output) leaves the same
    tree state as the eager prefill (reference decoding.py:143-185) for prompts that fill the rings
    partly or fully and reach 1 .. all 6 levels: B_hist, rg_hist for every level (beyond the
    horizon too), every V_ring slot (written or untouched) and the prefill logits (fp32)."""
    # (the prefill decoder itself: the graphed decoder's capture warm-ups then write position T)
    from dispatcher_hybrid.decoding import IncrementalDecoder, _FusedPrefillDecoder
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd, device=DEV)
    prompts = torch.randint(0, 250, (2, T), device=DEV, generator=torch.Generator(device=DEV).manual_seed(T))
    eager, fused = IncrementalDecoder(m), _FusedPrefillDecoder(m)
    le = eager.prefill(prompts)
    lf = fused.prefill(prompts)
    assert rel_err(lf, le) < 1e-5
    n = 0
    for ce, cf in zip(eager.caches, fused.caches):
        if hasattr(ce, "V_ring"):
            n += 1
            assert max_abs(cf.B_hist, ce.B_hist) < 1e-5        # layer 2 on: inputs differ by ulps
            assert max_abs(cf.rg_hist, ce.rg_hist) < 1e-5      # sigmoid: a few fp32 ulps
            assert max_abs(cf.V_ring, ce.V_ring) < 1e-5
    assert n == 2


def test_batched_graphed_and_fused_bf16():
    """reference tests/test_decoding.py:156-178 (bf16, 4 rows)."""
    from dispatcher_hybrid.decoding import (FusedGraphedHybridDecoder, GraphedHybridDecoder,
                                            IncrementalDecoder)
    cfgd, sd = tiny("tiny_a", scheme="reference")
    sd = dict(sd)
    m = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16)
    torch.manual_seed(0)
    prompts = torch.randint(0, 250, (4, 40), device=DEV)
    nexts = torch.randint(0, 250, (4, 6), device=DEV)

    def run(cls):
        dec = cls(m)
        out = [dec.prefill(prompts)[:, -1].float()]
        out += [dec.step(nexts[:, j]).float() for j in range(6)]
        return torch.stack(out, 1)

    ref = run(IncrementalDecoder)
    # the graphed decoder replays the eager decoder's own step: bitwise identical
    assert torch.equal(run(GraphedHybridDecoder), ref), "graphed batched must match eager batched exactly"
    got = run(FusedGraphedHybridDecoder)
    assert (got - ref).abs().max().item() < 1.0
    assert decisive_argmax_agree(got, ref)


def test_fast_generate_fused_equals_eager_greedy():
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd, device=DEV)
    g = golden("tiny_a")
    prompt = torch.from_numpy(g["gen"][:, :6]).to(DEV)
    n = g["gen"].shape[1] - 6
    fused = m.fast_generate(prompt, max_new_tokens=n, decoder="fused")
    eager = m.fast_generate(prompt, max_new_tokens=n, decoder="eager")
    assert torch.equal(fused, eager)
    assert np.array_equal(fused.cpu().numpy(), g["gen"])
    auto = m.fast_generate(prompt, max_new_tokens=n, decoder="auto")
    assert torch.equal(auto, eager)


@pytest.mark.parametrize("B", [1, 2])
def test_step_greedy_equals_argmax_of_step(B):
    """The device greedy loop (pick fused into the captured step; batch 1 through the vocabulary
    head's candidates, batch 2 through dh_argmax) yields the tokens argmax(step(tok)) yields, and
    tok_hist holds them at their positions."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    cfgd, sd = tiny("tiny_b")
    m = product_model(cfgd, sd, device=DEV)
    prompt = torch.randint(0, 250, (B, 9), device=DEV, generator=torch.Generator(device=DEV).manual_seed(B))
    ref_dec, dec = FusedGraphedHybridDecoder(m), FusedGraphedHybridDecoder(m)
    lg = ref_dec.prefill(prompt)[:, -1]
    ref = []
    for _ in range(20):
        tok = lg.argmax(-1)
        ref.append(tok)
        lg = ref_dec.step(tok)
    t0 = 9
    dec.greedy_start(dec.prefill(prompt)[:, -1])
    for _ in range(19):
        dec.step_greedy()
    got = dec.tok_hist[:, t0:t0 + 20]
    assert torch.equal(got, torch.stack(ref, 1))
    assert torch.equal(dec.token_buf, ref[-1])


def test_fast_generate_fused_sampling_support_and_reproducibility():
    """do_sample through the fused decoder draws on the device (dh_sample_topk): every generated
    token lies in the top-k set of the logits at its position (teacher-forced fp32 oracle forward
    over the generated sequence), and torch.manual_seed reproduces a run (eos: the test below)."""
    cfgd, sd = tiny("tiny_a")
    m = product_model(cfgd, sd, device=DEV)
    spec = te.Spec(m.config)
    prompt = torch.randint(0, cfgd["vocab_size"] - 1, (1, 12), generator=torch.Generator().manual_seed(1))
    k, T, n = 5, 0.7, 20
    torch.manual_seed(42)
    out = m.fast_generate(prompt.to(DEV), max_new_tokens=n, do_sample=True, temperature=T, top_k=k,
                          num_return_sequences=4, decoder="fused")
    torch.manual_seed(42)
    again = m.fast_generate(prompt.to(DEV), max_new_tokens=n, do_sample=True, temperature=T, top_k=k,
                            num_return_sequences=4, decoder="fused")
    assert torch.equal(out, again)
    assert out.shape == (4, 12 + n)
    logits = te.forward(sd, spec, out.cpu())                            # (4, 32, V) fp32
    live = torch.ones(4, dtype=torch.bool)     # a generated EOT is doc-masked only by the forward
    for t in range(12, 12 + n):
        l = logits[:, t - 1] / T
        kth = torch.topk(l, k, dim=-1).values[:, -1]
        tok = out[:, t].cpu()
        inside = l.gather(1, tok[:, None])[:, 0] >= kth - 1e-5
        assert bool((inside | ~live).all()), t
        live &= tok != cfgd["eot_token"]
    assert len({tuple(r) for r in out[:, 12:].tolist()}) > 1           # rows diverge


@pytest.mark.parametrize("mode", ["greedy", "sample_top1"])
def test_fast_generate_fused_eos_freezes_rows(mode):
    """reference tests/test_decoding.py:192-203 through the fused decoder (its eos branch: the
    device pick per step, host-side freezing): eos is row 0's first greedy token, so row 0 emits it
    at once and is padded with it while row 1 goes on; the result equals the eager decoder's with
    the same eos. sample_top1: the device sampler with top_k = 1 (its argmax)."""
    cfgd, sd = tiny("tiny_a", scheme="reference")
    m = product_model(cfgd, sd, device=DEV)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (2, 8), device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(11))
    eos = int(m.generate(ids[:1], max_new_tokens=1, do_sample=False)[0, -1])
    kw = dict(do_sample=True, top_k=1) if mode == "sample_top1" else {}
    out = m.fast_generate(ids, max_new_tokens=6, decoder="fused", eos_token_id=eos, **kw)
    assert int(out[0, 8]) == eos
    assert bool((out[0, 8:] == eos).all()), "finished row must be frozen at eos"
    assert out.shape[0] == 2 and 9 <= out.shape[1] <= 14
    eager = m.fast_generate(ids, max_new_tokens=6, decoder="eager", eos_token_id=eos)
    assert torch.equal(out, eager), (out.tolist(), eager.tolist())
    assert bool((out[1, 8:] != eos).any()) or out.shape[1] == 9


def test_generate_matches_fast_generate_on_gpu():
    """reference tests/test_decoding.py:89-95 and tests/test_parity.py:61-64 on the GPU: HF
    generate() (full recompute through the model's forward each token) on the product model yields
    the tokens greedy fast_generate yields through the eager and the fused decoders, and the same
    again with enable_fused_gates() (generate() then runs the fused forward)."""
    cfgd, sd = tiny("tiny_a", scheme="reference")
    m = product_model(cfgd, sd, device=DEV)
    V = cfgd["vocab_size"]
    ids = torch.tensor([[464 % V, 11844 % V, 286 % V, 262 % V]], device=DEV)
    a = m.generate(ids, max_new_tokens=12, do_sample=False)
    assert a.shape == (1, 16)
    assert torch.equal(a, m.fast_generate(ids, max_new_tokens=12, decoder="eager"))
    assert torch.equal(a, m.fast_generate(ids, max_new_tokens=12, decoder="fused"))
    m.enable_fused_gates()
    try:
        assert torch.equal(a, m.generate(ids, max_new_tokens=12, do_sample=False))
    finally:
        m.enable_fused_gates(False)


def test_fused_gates_beyond_add_rmsnorm_width_fp32():
    """An fp32 model wider than dh_add_rmsnorm takes (d = 4224 > 4096 fp32 elements per row): with
    enable_fused_gates() the forward takes the block-by-block loop (the mixer still on the fused
    kernels) instead of raising mid-forward, and equals the eager forward (rel <= 1e-4)."""
    from dispatcher_hybrid.fused_gates import add_rmsnorm_fits
    cfgd = dict(vocab_size=256, d_model=4224, num_heads=33, dim_feedforward=256, num_layers=1, max_len=64,
                attn_layers=(), attn_window=0, doc_reset=False, eot_token=255)
    assert not add_rmsnorm_fits(4224, torch.float32) and add_rmsnorm_fits(4224, torch.bfloat16)
    sd = make_state_dict(cfgd, 3)
    m = product_model(cfgd, sd, device=DEV)
    ids = torch.randint(0, 255, (2, 40), device=DEV, generator=torch.Generator(device=DEV).manual_seed(2))
    with torch.no_grad():
        ref = m(ids).logits
        m.enable_fused_gates()
        try:
            x = m.embedding(ids)
            assert not m._fused_norm_ok(x, False)
            got = m(ids).logits
        finally:
            m.enable_fused_gates(False)
    r = rel_err(got, ref)
    print(f"d=4224 fp32 fused vs eager rel={r:.2e}", flush=True)
    assert r <= 1e-4


def test_fused_decoder_context_exhausted_raises():
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    cfgd, sd = tiny("tiny_b")
    m = product_model(cfgd, sd, device=DEV)
    dec = FusedGraphedHybridDecoder(m)
    dec.prefill(torch.randint(0, 250, (cfgd["max_len"] - 1,), device=DEV))
    dec.step(torch.tensor(3, device=DEV))
    with pytest.raises(ValueError, match="context exhausted"):
        dec.step(torch.tensor(3, device=DEV))


# --------------------------------------------------------------------------------------------
# release shapes (292M, bf16)
# --------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def release_models():
    """292M random init (reference scheme, but W1s ~ N(0, 0.02) so lag indexing is exercised),
    in bf16 and fp32 on the GPU."""
    cfgd = RELEASE_CONFIG
    sd = make_state_dict(cfgd, 0, scheme="reference")
    g = torch.Generator().manual_seed(1)
    for k in list(sd):
        if k.endswith("gate_hidden_src.weight"):
            sd[k] = torch.randn(sd[k].shape, generator=g) * 0.02
    m32 = product_model(cfgd, sd, device=DEV)
    m16 = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16)
    return cfgd, m32, m16


def test_release_prefill_fused_gates_tolerances(release_models):
    """C2: T=1024 prefill with a doc boundary. fp32: fused vs eager rel <= 1e-4. bf16:
    helpers.bf16_vs_truth, with the eager path's same-rounding floor measured here."""
    cfgd, m32, m16 = release_models
    torch.manual_seed(2)
    ids = torch.randint(0, cfgd["vocab_size"], (1, 1024), device=DEV)
    ids[0, 300] = cfgd["eot_token"]                       # exercise the doc-reset mask
    with torch.no_grad():
        e32 = m32(ids).logits.float()
        f32 = m32.enable_fused_gates()(ids).logits.float()
        m32.enable_fused_gates(False)
        e16 = m16(ids).logits.float()
        with fp32_product_accumulation():
            a16 = m16(ids).logits.float()
        f16 = m16.enable_fused_gates()(ids).logits.float()
        m16.enable_fused_gates(False)
    r32 = rel_err(f32, e32)
    print(f"C2 fp32 rel={r32:.2e}", flush=True)
    assert r32 <= 1e-4
    bf16_vs_truth(f16, e16, e32, "C2 bf16", alt16=a16)


def test_release_graphed_forward_equals_fused_forward(release_models):
    """graphed_logits (the C2 prefill as one HIP graph replay) against the fused forward it captured,
    bit for bit: several replays, new token ids between them (one with an EOT, so the doc-reset mask
    changes), the eager forward run between replays, and a second shape with its own graph."""
    cfgd, m32, m16 = release_models
    g = torch.Generator(device=DEV).manual_seed(5)
    m16.enable_fused_gates()
    try:
        with torch.no_grad():
            for rep in range(4):
                ids = torch.randint(0, cfgd["vocab_size"], (1, 1024), device=DEV, generator=g)
                if rep == 2:
                    ids[0, 500] = cfgd["eot_token"]
                print(f"graphed forward replay {rep}", flush=True)
                got = m16.graphed_logits(ids).clone()
                torch.cuda.synchronize()
                ref = m16(ids).logits
                torch.cuda.synchronize()
                assert torch.equal(got, ref), f"replay {rep} differs from the fused forward"
            ids2 = torch.randint(0, cfgd["vocab_size"], (2, 256), device=DEV, generator=g)
            got2 = m16.graphed_logits(ids2).clone()
            assert torch.equal(got2, m16(ids2).logits)
            assert torch.equal(m16.graphed_logits(ids), m16(ids).logits)   # the first shape's graph again
    finally:
        m16.release_graphs()
        m16.enable_fused_gates(False)


def test_release_gate_preacts_bf16_per_layer(release_models):
    """Per-layer gate pre-activations (the fused op's outputs) against the eager formula on the
    same bf16 A and B (C5-style check at B=2, T=2048, doc mask on), bounded in bf16 ulps at the eager
    rounding points (helpers.preact_bound: the eager path rounds twice, product then bias add, the
    fused op once)."""
    from dispatcher_hybrid.modeling_dispatcher import level_gate_matmul
    cfgd, m32, m16 = release_models
    torch.manual_seed(4)
    ids = torch.randint(0, cfgd["vocab_size"], (2, 2048), device=DEV)
    ids[:, 700] = cfgd["eot_token"]
    caps = {}
    hooks = []
    mx = m16.blocks[3].mixer
    hooks.append(mx.register_forward_pre_hook(lambda mod, inp: caps.__setitem__("xm", inp)))
    with torch.no_grad():
        m16(ids)
    for hk in hooks:
        hk.remove()
    x, mask = caps["xm"]
    with torch.no_grad():
        A, Bs = mx.gate_hidden(x), mx.gate_hidden_src(x)
        n_lv = 12
        m3 = mask[..., :n_lv]
        fused = torch.ops.dispatcher.gate_preacts_fwd(A, Bs, mx.gate_out, mx.forget_out, mx.reset_out,
                                                      mx.gate_out_bias, mx.forget_out_bias,
                                                      mx.reset_out_bias, n_lv, m3)
        lagged = torch.stack([torch.roll(Bs, shifts=1 << l, dims=1) for l in range(n_lv)], dim=2)
        hidden = torch.relu(A.unsqueeze(2) + lagged * m3.unsqueeze(-1)) ** 2
        for got, (W, b) in zip(fused, mx._gate_params()):
            ref = level_gate_matmul(hidden, W[:n_lv]) + b[:n_lv]
            diff = (got.float() - ref.float()).abs()
            bound = preact_bound(got, ref, b[:n_lv].float().expand_as(ref), level_gate_matmul(hidden, W[:n_lv].abs()))
            print(f"gate preacts bf16 max|d|={diff.max().item():.4f} (|ref| max "
                  f"{ref.abs().max().item():.3f}), worst |d|/bound={(diff / bound).max().item():.3f}", flush=True)
            assert bool((diff <= bound).all())


def test_release_decode_fused_tolerances(release_models):
    """C3-style decode: prefill 1024 + 16 steps. fp32: fused vs eager decoder rel <= 1e-4.
    bf16: see _bf16_vs_truth (truth = the fp32 eager decoder)."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    cfgd, m32, m16 = release_models
    torch.manual_seed(3)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (1, 1040), device=DEV)

    def run(m, cls):
        dec = cls(m)
        dec.prefill(ids[:, :1024])
        return torch.stack([dec.step(ids[:, t]).float() for t in range(1024, 1040)], 1)

    e32, f32 = run(m32, IncrementalDecoder), run(m32, FusedGraphedHybridDecoder)
    r = rel_err(f32, e32)
    print(f"C3 fp32 rel={r:.2e}", flush=True)
    assert r <= 1e-4
    bf16_vs_truth(run(m16, FusedGraphedHybridDecoder), run(m16, IncrementalDecoder), e32, "C3 bf16")


def test_release_decode_step_bf16_layer_local(release_models):
    """One tree layer's decode step (bf16) against the eager step's arithmetic on the identical
    state: the mixer output Y within 3e-2 max-abs."""
    from dispatcher_hybrid import fused_step
    from dispatcher_hybrid.decoding import IncrementalDecoder
    cfgd, m32, m16 = release_models
    torch.manual_seed(5)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (2, 900), device=DEV)
    dec = IncrementalDecoder(m16)
    dec.prefill(ids)
    blk, cache = m16.blocks[0], dec.caches[0]
    mx = blk.mixer
    t = ids.shape[1]
    with torch.no_grad():
        x = torch.randn(2, cfgd["d_model"], device=DEV, dtype=torch.bfloat16)
        h1 = blk.norm1(x)
        A, Bt, V0 = mx.gate_hidden(h1), mx.gate_hidden_src(h1), mx.linear_in(h1)
        cache.B_hist[:, t] = Bt
        state = (cache.rg_hist.clone(), cache.V_ring.clone())
        Y = torch.empty_like(V0)
        t_buf = torch.full((1,), t, dtype=torch.long, device=DEV)
        fused_step.decode_mixer_step(A, cache.B_hist, mx.gate_out, mx.forget_out, mx.reset_out,
                                     mx.gate_out_bias, mx.forget_out_bias, mx.reset_out_bias, t_buf,
                                     cache.rg_hist, cache.V_ring, V0, Y)
        # eager arithmetic of the same step (reference decoding.py:193-220), on the saved state
        rg_hist, V_ring = state
        L, H, hd = cache.L, cache.H, cache.hd
        lev = torch.arange(L, device=DEV)
        src = t - torch.pow(2, lev)
        okf = (src >= 0).view(1, L, 1)
        src_c = src.clamp(min=0)
        hid = torch.relu(A.unsqueeze(1) + cache.B_hist[:, src_c] * okf) ** 2
        from dispatcher_hybrid.modeling_dispatcher import level_gate_matmul
        g = [level_gate_matmul(hid.unsqueeze(1), W)[:, 0] + b for W, b in mx._gate_params()]
        i_, f_ = torch.sigmoid(g[0]) * okf, torch.sigmoid(g[1]) * okf + (~okf).to(x.dtype)
        msg = rg_hist[:, src_c, lev].unsqueeze(-1) * V_ring[:, cache.offsets + (src_c & cache.masks)].view(2, L, H, hd)
        V = V0.view(2, H, hd)
        for l in range(L):
            V = f_[:, l].unsqueeze(-1) * V + i_[:, l].unsqueeze(-1) * msg[:, l]
    gap = (Y.float() - V.reshape(2, -1).float()).abs().max().item()
    print(f"decode step bf16 Y max|d|={gap:.4f} (|Y| max {V.abs().max().item():.3f})", flush=True)
    assert gap <= 3e-2
