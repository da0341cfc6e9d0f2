"""Next-token selection on the device, against the calls it replaces in fast_generate (reference
dispatcher_hybrid/modeling_dispatcher.py:426-441).

dh_argmax vs torch.argmax: same index bit for bit, including ties (first index) and NaN (first NaN).
dh_sample_topk vs logits.float() / T, torch.topk masking, softmax, multinomial: its random stream
is not torch's, so it is checked by (1) support -- every draw lies in the set torch's own top-k
mask keeps, ties at the k-th value included -- and (2) distribution -- a chi-square test of many
draws against the float64 softmax of the masked logits (6-sigma bound; the draws are a fixed
function of the seeds, so the outcome is deterministic)."""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,V", [(1, 50257), (16, 50257), (3, 7), (2, 1024), (5, 65536), (1, 1)])
def test_argmax_matches_torch(B, V, dtype):
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(B * 1000 + V)
    x = torch.randn(B, V, device=DEV, generator=g).to(dtype)
    got = fused_step.argmax_tokens(x)
    torch.cuda.synchronize()
    assert torch.equal(got, x.argmax(-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_ties_nan_and_strided_rows(dtype):
    from dispatcher_hybrid import fused_step
    V = 5000
    x = torch.zeros(4, V + 3, device=DEV, dtype=dtype)[:, :V]          # row stride V + 3
    x[0, 17] = 2.0
    x[0, 4000] = 2.0                                                     # tie: first index wins
    x[1, :] = -1.0
    x[1, 4999] = float("nan")
    x[1, 3] = float("nan")                                               # first NaN wins
    x[2, 1234] = float("inf")
    x[3, :] = -float("inf")                                              # all equal: index 0
    got = fused_step.argmax_tokens(x)
    torch.cuda.synchronize()
    assert got.tolist() == [17, 3, 1234, 0]
    assert torch.equal(got, x.argmax(-1))


def _cand_records(pairs):
    """(value, index) pairs as the 8-byte candidate records of dh_decode_gemv (float, int32)."""
    import struct
    raw = b"".join(struct.pack("<fi", v, i) for v, i in pairs)
    return torch.frombuffer(bytearray(raw), dtype=torch.int64).to(DEV).view(1, -1)


def test_argmax_reduce_order_and_history():
    """The candidate reduce of the fused greedy pick: torch.argmax's order (larger value, NaN above
    all, lowest index on ties) over up to 8192 records, and the optional history write at t_buf."""
    from dispatcher_hybrid import fused_step
    out = torch.empty(1, dtype=torch.long, device=DEV)
    cases = [([(1.0, 5), (3.0, 9), (3.0, 2), (-1.0, 0)], 2),                 # tie: lowest index
             ([(float("-inf"), 7), (float("nan"), 40), (5.0, 1), (float("nan"), 12)], 12),   # first NaN
             ([(float(k % 97), k) for k in range(8192)], 96)]               # 8192 records, first 96
    for pairs, want in cases:
        fused_step.argmax_reduce(_cand_records(pairs), out)
        torch.cuda.synchronize()
        assert int(out) == want
    hist = torch.full((1, 10), -1, dtype=torch.long, device=DEV)
    t_buf = torch.tensor([5], device=DEV)
    fused_step.argmax_reduce(_cand_records([(2.0, 31), (1.0, 4)]), out, t_buf, hist)
    t_buf.fill_(12)                                                       # past the history: no write
    fused_step.argmax_reduce(_cand_records([(2.0, 8)]), out, t_buf, hist)
    torch.cuda.synchronize()
    assert hist[0, 5].item() == 31 and int(out) == 8
    assert int((hist != -1).sum()) == 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lm_head_candidates_give_torch_argmax(dtype):
    """dh_decode_gemv's per-workgroup candidates (the release vocabulary head shape) reduced by
    dh_argmax_reduce equal torch.argmax of the logits the same launch wrote: random rows, two tied
    maximal rows (the lower wins), and a NaN row (NaN wins)."""
    from dispatcher_hybrid import fused_step
    V, K = 50257, 1024
    g = torch.Generator(device=DEV).manual_seed(9)
    W = (torch.randn(V, K, device=DEV, generator=g) / K ** 0.5).to(dtype)
    x = torch.randn(1, K, device=DEV, generator=g).to(dtype)
    w = torch.ones(K, device=DEV, dtype=dtype)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    for variant in ("random", "tie", "nan"):
        if variant == "tie":
            W[40000] = W[123] = x[0] * 3                                    # equal maximal rows
        if variant == "nan":
            W[31000, 5] = float("nan")
        logits = torch.empty(1, V, device=DEV, dtype=dtype)
        cand = fused_step.candidate_buffer(dtype, V, K, 1, DEV)
        fused_step.decode_gemv(x, [(W, logits, V, 0)], t_buf, norm_weight=w, argmax_cand=cand)
        out = fused_step.argmax_reduce(cand, torch.empty(1, dtype=torch.long, device=DEV))
        torch.cuda.synchronize()
        assert int(out) == int(logits.argmax(-1)), variant
        if variant == "tie":
            assert int(out) == 123
        if variant == "nan":
            assert int(out) == 31000


def test_argmax_rejects_bad_shapes():
    from dispatcher_hybrid import fused_step
    with pytest.raises(ValueError):
        fused_step.argmax_tokens(torch.zeros(3, device=DEV))
    with pytest.raises(ValueError):
        fused_step.argmax_tokens(torch.zeros(2, 8, device=DEV), out=torch.zeros(3, dtype=torch.long, device=DEV))


def test_argmax_large_vocabulary():
    """Vocabularies far past one workgroup's slice (200k entries, 98 slices)."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(3, 200003, device=DEV, generator=g)
    x[1, 199999] = 100.0
    assert torch.equal(fused_step.argmax_tokens(x), x.argmax(-1))


def _kept_and_probs(logits, temperature, top_k):
    """The reference's masking and softmax (modeling_dispatcher.py:454-459) on the same device."""
    l = logits.float() / temperature
    if top_k is not None:
        kth = torch.topk(l, top_k, dim=-1).values[:, -1:]
        l = l.masked_fill(l < kth, float("-inf"))
    return torch.isfinite(l), torch.softmax(l.double(), dim=-1)


def _chi2_ok(draws, p, label):
    """draws: int64 tokens of one distribution p (V,) float64. Categories with expected count < 5
    are pooled. Passes when chi2 < df + 6 sqrt(2 df)."""
    n = draws.numel()
    obs = torch.bincount(draws.cpu(), minlength=p.numel()).double()
    exp = p.cpu() * n
    big = exp >= 5
    o = torch.cat([obs[big], obs[~big].sum().view(1)])
    e = torch.cat([exp[big], exp[~big].sum().view(1)])
    keep = e > 0
    o, e = o[keep], e[keep]
    chi2 = float(((o - e) ** 2 / e).sum())
    df = max(int(keep.sum()) - 1, 1)
    bound = df + 6 * math.sqrt(2 * df)
    print(f"{label}: n={n} categories={df + 1} chi2={chi2:.1f} bound={bound:.1f}", flush=True)
    assert chi2 < bound, (label, chi2, bound)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sample_topk_distribution_with_ties(dtype):
    """top_k = 50 of 1000 at T = 0.8, with four logits tied at the 50th value: every draw is kept by
    torch's mask (all four ties included) and the frequencies follow its softmax."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(7)
    V, k, T, rows = 1000, 50, 0.8, 8192
    base = torch.randn(V, device=DEV, generator=g) * 2
    order = base.argsort(descending=True)
    base[order[k - 2:k + 2]] = float(base[order[k - 2]])               # ties across the boundary
    logits = base.to(dtype).expand(rows, V).contiguous()
    kept, p = _kept_and_probs(logits[:1], T, k)
    assert int(kept.sum()) >= k + 2
    off = torch.zeros(1, dtype=torch.long, device=DEV)
    draws = []
    for step in range(4):
        off.fill_(1000 + step)
        draws.append(fused_step.sample_tokens(logits, T, k, seed=123, offset=off))
    d = torch.cat(draws)
    torch.cuda.synchronize()
    assert bool(kept[0, d].all()), "a draw outside the top-k set"
    tied = order[k - 2:k + 2]
    assert all(int((d == i).sum()) > 0 for i in tied.tolist())       # every tie can be drawn
    _chi2_ok(d, p[0], f"top-k {dtype}")


def test_sample_full_softmax_and_temperature():
    """No top-k (every logit kept) at T = 1.3 over 300 logits."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(8)
    V, T, rows = 300, 1.3, 16384
    base = torch.randn(V, device=DEV, generator=g) * 1.5
    logits = base.expand(rows, V).contiguous()
    _, p = _kept_and_probs(logits[:1], T, None)
    d = fused_step.sample_tokens(logits, T, None, seed=99, offset=None)
    torch.cuda.synchronize()
    assert int(d.min()) >= 0 and int(d.max()) < V
    _chi2_ok(d, p[0], "full softmax")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sample_signed_zero_tie_and_minus_inf(dtype):
    """The kth value is +0.0 and other logits are -0.0: torch's mask (l < kth) keeps both signs, so
    every zero is drawable. -inf logits are never drawn, also when top_k reaches into them."""
    from dispatcher_hybrid import fused_step
    V, rows = 3000, 8192
    base = torch.full((V,), -5.0, device=DEV)
    base[10:20] = 1.0
    base[100:150:2] = 0.0
    base[101:151:2] = -0.0
    logits = base.to(dtype).expand(rows, V).contiguous()
    k = 11                                              # 10 ones, then the zeros tie at the kth
    kept, p = _kept_and_probs(logits[:1], 0.7, k)
    assert int(kept.sum()) == 10 + 50
    d = fused_step.sample_tokens(logits, 0.7, k, seed=3, offset=None)
    torch.cuda.synchronize()
    assert bool(kept[0, d].all()), "a draw outside torch's kept set"
    zeros = d[(d >= 100) & (d < 150)]
    assert int((zeros % 2 == 1).sum()) > 0 and int((zeros % 2 == 0).sum()) > 0   # both signs drawn
    _chi2_ok(d, p[0], f"signed zeros {dtype}")
    inf = torch.full((4, 200), float("-inf"), device=DEV)
    inf[:, :3] = torch.tensor([0.5, -1.0, 2.0], device=DEV)
    inf = inf.to(dtype)
    d2 = fused_step.sample_tokens(inf, 1.0, 50, seed=1, offset=None)
    torch.cuda.synchronize()
    assert int(d2.max()) < 3, "a -inf logit was drawn"


@pytest.mark.parametrize("V,k", [(5000, 2000), (50257, 50)])
def test_sample_wide_top_k_and_all_ties(V, k):
    """top_k > 1024 (the kth found by the exact key-space search) and a row of one repeated value
    (every element ties with the kth: all of them kept, drawn uniformly)."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(V)
    rows = 4096
    if V == 5000:
        base = torch.randn(V, device=DEV, generator=g)
    else:
        base = torch.full((V,), 0.75, device=DEV)
    logits = base.to(torch.bfloat16).expand(rows, V).contiguous()
    kept, p = _kept_and_probs(logits[:1], 1.0, k)
    d = fused_step.sample_tokens(logits, 1.0, k, seed=5, offset=None)
    torch.cuda.synchronize()
    assert bool(kept[0, d].all())
    if V == 5000:
        _chi2_ok(d, p[0], "top-k 2000")
    else:
        assert int(kept.sum()) == V
        assert d.unique().numel() > rows * 0.9                           # ~uniform over 50257


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sample_release_vocab_support(dtype):
    """The C4 setting: 16 rows of 50257 logits, T = 0.8, top-k 50, 32 steps keyed by an advancing
    device position: every draw inside its row's top-k set, and the draws vary."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(3)
    logits = (torch.randn(16, 50257, device=DEV, generator=g) * 3).to(dtype)
    kept, _ = _kept_and_probs(logits, 0.8, 50)
    pos = torch.full((1,), 3840, dtype=torch.long, device=DEV)
    seen = []
    for _ in range(32):
        d = fused_step.sample_tokens(logits, 0.8, 50, seed=2024, offset=pos)
        seen.append(d.clone())
        pos += 1
    d = torch.stack(seen)
    torch.cuda.synchronize()
    assert bool(kept.gather(1, d.T).all())
    assert d.unique().numel() > 50


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [50257, 7, 1025])
def test_sample_last_element_of_odd_rows(dtype, V):
    """Odd V, the released vocabulary included: the row's last element (the EOT token at V = 50257)
    sits in a dword whose upper half lies past the row. With logit[V-1] far above the rest every
    draw must be V-1 (top_k 1, 50 and the full softmax), in every row of a batch (rows start at
    odd element offsets) and for the row-strided argmax as well; the same with the maximum one
    before the end and the last element lowest, so the byte past the row is never taken as an
    element."""
    from dispatcher_hybrid import fused_step
    B = 5
    g = torch.Generator(device=DEV).manual_seed(V)
    x = torch.randn(B, V, device=DEV, generator=g)
    x[:, V - 1] = 40.0
    x = x.to(dtype)
    off = torch.tensor([9], dtype=torch.long, device=DEV)
    for k in (1, min(50, V), None):
        for seed in range(16):
            tok = fused_step.sample_tokens(x, temperature=0.8, top_k=k, seed=seed, offset=off)
            assert bool((tok == V - 1).all()), (k, seed, tok.tolist())
    assert bool((fused_step.argmax_tokens(x) == V - 1).all())
    if V > 2:
        y = torch.randn(B, V, device=DEV, generator=g)
        y[:, V - 2], y[:, V - 1] = 40.0, -40.0
        y = y.to(dtype)
        for k in (1, 2, None):
            tok = fused_step.sample_tokens(y, temperature=1.0, top_k=k, seed=3, offset=off)
            assert bool((tok == V - 2).all()), (k, tok.tolist())


def test_sample_deterministic_and_keyed():
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(4)
    logits = torch.randn(64, 4000, device=DEV, generator=g)
    o1 = torch.full((1,), 11, dtype=torch.long, device=DEV)
    o2 = torch.full((1,), 12, dtype=torch.long, device=DEV)
    a = fused_step.sample_tokens(logits, 1.0, 100, seed=1, offset=o1)
    b = fused_step.sample_tokens(logits, 1.0, 100, seed=1, offset=o1)
    c = fused_step.sample_tokens(logits, 1.0, 100, seed=1, offset=o2)
    e = fused_step.sample_tokens(logits, 1.0, 100, seed=2, offset=o1)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert not torch.equal(a, c) and not torch.equal(a, e)


@pytest.mark.parametrize("dtype,k", [(torch.float32, 100), (torch.bfloat16, 50), (torch.bfloat16, None)])
def test_sample_history_write(dtype, k):
    """dh_sample_topk_hist: the same draws as dh_sample_topk, each row's token also stored at
    hist[b, offset] (rows of stride 37 > L = 30), every other history entry untouched; an offset
    at or past L writes no history."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(9)
    logits = torch.randn(16, 50257, device=DEV, generator=g).to(dtype)
    base = torch.randint(0, 1000, (16, 37), device=DEV, generator=g)
    for pos in (0, 17, 29, 30, 31):
        off = torch.full((1,), pos, dtype=torch.long, device=DEV)
        ref = fused_step.sample_tokens(logits, 0.8, k, seed=5, offset=off)
        hist = base.clone()
        got = fused_step.sample_tokens(logits, 0.8, k, seed=5, offset=off, hist=hist[:, :30])
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        want = base.clone()
        if pos < 30:
            want[:, pos] = ref
        assert torch.equal(hist, want), pos


@pytest.mark.parametrize("dtype,k", [(torch.bfloat16, 50), (torch.bfloat16, None), (torch.float32, 50),
                                     (torch.float32, 2000)])
def test_sample_misaligned_rows(dtype, k):
    """Rows that start off 16-byte alignment (every element offset 0..7 past it: views into a wider
    tensor, as the odd rows of a (B, 50257) bf16 tensor are) are read from the aligned address below
    them and shifted into place: the same draws as the same values in 16-byte aligned rows, bit for
    bit, on the bf16 top-k kernel and the general one (no top-k, or k > 1024, or fp32)."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(31)
    B, V = 8, 50257
    big = torch.randn(B, V + 16, device=DEV, generator=g).to(dtype)
    off = torch.full((1,), 123, dtype=torch.long, device=DEV)
    aligned = torch.zeros(B, V + 7, device=DEV, dtype=dtype)[:, :V]
    assert aligned.stride(0) % 8 == 0 and aligned.data_ptr() % 16 == 0
    for o in range(8):
        view = big[:, o:o + V]                     # row b starts (b (V + 16) + o) elements in
        aligned.copy_(view)
        got = fused_step.sample_tokens(view, 0.8, k, seed=9, offset=off)
        ref = fused_step.sample_tokens(aligned, 0.8, k, seed=9, offset=off)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), o


def test_sample_top1_and_tiny_temperature_are_argmax():
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(6)
    logits = torch.randn(32, 50257, device=DEV, generator=g).to(torch.bfloat16)
    ref = logits.argmax(-1)
    top1 = fused_step.sample_tokens(logits, 0.9, 1, seed=3)
    cold = fused_step.sample_tokens(logits, 1e-6, None, seed=3)
    torch.cuda.synchronize()
    uniq = [(logits[r] == logits[r].max()).sum().item() == 1 for r in range(32)]
    for r in range(32):
        if uniq[r]:
            assert int(top1[r]) == int(ref[r]) and int(cold[r]) == int(ref[r])


def test_sample_rejects_bad_arguments():
    from dispatcher_hybrid import fused_step
    x = torch.zeros(2, 10, device=DEV)
    with pytest.raises(ValueError, match="top_k"):
        fused_step.sample_tokens(x, 1.0, 11)
    with pytest.raises(ValueError, match="temperature"):
        fused_step.sample_tokens(x, 0.0, 5)
    with pytest.raises(ValueError, match="65536"):
        fused_step.sample_tokens(torch.zeros(1, 70000, device=DEV), 1.0, 5)
    hist = torch.zeros(2, 8, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="offset"):
        fused_step.sample_tokens(x, 1.0, 5, hist=hist)
    off = torch.zeros(1, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="hist"):
        fused_step.sample_tokens(x, 1.0, 5, offset=off, hist=hist[:1])


@pytest.mark.parametrize("batch", [1, 16])
def test_step_sample_matches_step_then_sample(batch):
    """FusedGraphedHybridDecoder.step_sample (the sampler recorded as the last launch of the graphed
    step, the sampled token feeding the next replay on the device) against step() followed by
    sample_tokens(logits, T, k, seed, t_buf) per token, the loop fast_generate ran before: the same
    logits after every step and the same tokens; fast_generate's sampling branch returns them."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    from dispatcher_hybrid import fused_step
    from helpers import product_model
    from weights import make_state_dict
    cfg = dict(vocab_size=2048, d_model=512, num_heads=8, dim_feedforward=1024, num_layers=4, max_len=256,
               attn_layers=(2, 4), attn_window=64, doc_reset=True, eot_token=2047)
    m = product_model(cfg, make_state_dict(cfg, 7), device=DEV, dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(21)
    prompt = torch.randint(0, 2047, (1, 24), device=DEV, generator=g).expand(batch, -1).contiguous()
    print(f"step_sample: batch {batch}", flush=True)
    da, db = FusedGraphedHybridDecoder(m), FusedGraphedHybridDecoder(m)
    la, lb = da.prefill(prompt)[:, -1], db.prefill(prompt)[:, -1]
    t0 = da.t
    da.sample_start(la, 0.8, 50, 77)
    tok = fused_step.sample_tokens(lb, 0.8, 50, 77, db.t_buf)
    toks = [tok.clone()]
    for i in range(30):
        da.step_sample()
        lb = db.step(tok)
        assert torch.equal(da.logits_out, lb), f"logits differ at step {i}"
        tok = fused_step.sample_tokens(lb, 0.8, 50, 77, db.t_buf)
        toks.append(tok.clone())
    assert torch.equal(da.tok_hist[:, t0:t0 + 31], torch.stack(toks, 1))
    assert torch.equal(da.token_buf, tok) and da.t == db.t
    # fast_generate's sampling branch (no eos): the seed comes from torch's generator
    torch.manual_seed(3)
    out = m.fast_generate(prompt, max_new_tokens=12, do_sample=True, temperature=0.8, top_k=50, decoder="fused")
    torch.manual_seed(3)
    seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    dc = FusedGraphedHybridDecoder(m)
    lc = dc.prefill(prompt)[:, -1]
    ref = []
    for i in range(12):
        tk = fused_step.sample_tokens(lc, 0.8, 50, seed, dc.t_buf)
        ref.append(tk.clone())
        if i < 11:
            lc = dc.step(tk)
    assert torch.equal(out[:, 24:], torch.stack(ref, 1))
