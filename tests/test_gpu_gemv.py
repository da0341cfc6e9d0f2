"""dh_decode_gemv (fused RMSNorm / projections / residual / SwiGLU of the decode step) against torch
evaluated in float64 on the same inputs, with the eager path's rounding points reproduced for bf16
(reference dispatcher_hybrid/decoding.py:473-488, modeling_dispatcher.py:196-197, 207-212)."""

import pytest
import torch
import torch.nn.functional as F

from helpers import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rnd(x, dt):
    return x.to(dt).double()


def _norm(x, g, dt):
    eps = torch.finfo(torch.float32).eps                # nn.RMSNorm(eps=None) for fp32 and bf16 inputs
    xd = x.double()
    h = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * g.double()
    return _rnd(h, dt)


# (B, K): K = 176 and 352 are the tiny test models' widths (not multiples of 64 elements)
CASES = [(1, 1024), (3, 512), (16, 1024), (70, 256), (2, 176), (5, 352), (8, 3072)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("scale", [1.0, 0.02])
def test_norm_matches_torch_rms_norm(dtype, scale):
    """An identity weight makes the output the normalised row itself, which must equal torch's own
    F.rms_norm(eps=None) on the device; scale 0.02 is the embedding scale of a fresh model, where
    the default epsilon is not negligible."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(17)
    B, K = 4, 1024
    x = (torch.randn(B, K, device=DEV, generator=g) * scale).to(dtype)
    w = torch.rand(K, device=DEV, generator=g).add(0.5).to(dtype)
    eye = torch.eye(K, device=DEV, dtype=dtype)
    out = torch.empty(B, K, device=DEV, dtype=dtype)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(x, [(eye, out, K, 0)], t_buf, norm_weight=w)
    torch.cuda.synchronize()
    ref = F.rms_norm(x, (K,), w)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -20
    assert bool(((out.double() - ref.double()).abs() <= ulp * ref.double().abs() + 1e-30).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,K", CASES)
def test_norm_three_segments_with_position_row(B, K, dtype):
    from dispatcher_hybrid import fused_step
    print(f"gemv segments B={B} K={K} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(B * 7 + K)
    x = (torch.randn(B, K, device=DEV, generator=g) * 0.02).to(dtype)
    w = torch.rand(K, device=DEV, generator=g).add(0.5).to(dtype)
    Ws = [(torch.randn(n, K, device=DEV, generator=g) / K ** 0.5).to(dtype) for n in (K, 96, K)]
    o0 = torch.full((B, K), 7.0, device=DEV, dtype=dtype)
    o1 = torch.full((B, 96), 7.0, device=DEV, dtype=dtype)
    Tmax = 9
    hist = torch.full((B, Tmax, K), 7.0, device=DEV, dtype=dtype)
    t_buf = torch.full((1,), 5, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(x, [(Ws[0], o0, K, 0), (Ws[1], o1, 96, 0), (Ws[2], hist, Tmax * K, K)], t_buf,
                           norm_weight=w)
    torch.cuda.synchronize()
    h = _norm(x, w, dtype)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_err(o0, _rnd(h @ Ws[0].double().T, dtype)) < tol
    assert rel_err(o1, _rnd(h @ Ws[1].double().T, dtype)) < tol
    assert rel_err(hist[:, 5], _rnd(h @ Ws[2].double().T, dtype)) < tol
    untouched = torch.cat([hist[:, :5], hist[:, 6:]], 1)
    assert bool((untouched == 7.0).all()), "only row t of the history may be written"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,K", CASES)
def test_residual_in_place(B, K, dtype):
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(B + K)
    N = 640
    v = torch.randn(B, K, device=DEV, generator=g).to(dtype)
    W = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(dtype)
    x = torch.randn(B, N, device=DEV, generator=g).to(dtype)
    x0 = x.clone()
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(v, [(W, x, N, 0)], t_buf, resid=x)          # x += W v, in place
    torch.cuda.synchronize()
    ref = _rnd(_rnd(v.double() @ W.double().T, dtype) + x0.double(), dtype)
    assert rel_err(x, ref) < (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,K,ff", [c + (352,) for c in CASES] + [(1, 1024, 2816), (16, 1024, 2816)])
def test_norm_swiglu(B, K, ff, dtype):
    """ff = 2816 is the released FFN width: two weight rows per output with two rows per wave."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(3 * B + K)
    x = torch.randn(B, K, device=DEV, generator=g).to(dtype)
    w = torch.rand(K, device=DEV, generator=g).add(0.5).to(dtype)
    Wg = (torch.randn(ff, K, device=DEV, generator=g) / K ** 0.5).to(dtype)
    Wu = (torch.randn(ff, K, device=DEV, generator=g) / K ** 0.5).to(dtype)
    out = torch.empty(B, ff, device=DEV, dtype=dtype)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(x, [(Wg, out, ff, 0), (Wu, out, ff, 0)], t_buf, norm_weight=w, swiglu=True)
    torch.cuda.synchronize()
    h = _norm(x, w, dtype)
    gate, up = _rnd(h @ Wg.double().T, dtype), _rnd(h @ Wu.double().T, dtype)
    ref = _rnd(_rnd(F.silu(gate), dtype) * up, dtype)
    assert rel_err(out, ref) < (1e-5 if dtype == torch.float32 else 1.5e-2)


@pytest.mark.parametrize("B", [1, 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_embedding_gather_rows(dtype, B):
    """x_rows / resid_rows: the first decode launch reads the token rows of the embedding."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(11)
    V, K, N = 300, 256, 256
    emb = torch.randn(V, K, device=DEV, generator=g).to(dtype)
    tok = torch.tensor([299, 3, 0, 3, 150], device=DEV)[:B]
    W = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(dtype)
    w = torch.rand(K, device=DEV, generator=g).add(0.5).to(dtype)
    out = torch.empty(B, N, device=DEV, dtype=dtype)
    res = torch.empty(B, N, device=DEV, dtype=dtype)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(emb, [(W, out, N, 0)], t_buf, norm_weight=w, x_rows=tok)
    fused_step.decode_gemv(out, [(W, res, N, 0)], t_buf, resid=emb, resid_rows=tok)
    torch.cuda.synchronize()
    h = _norm(emb[tok], w, dtype)
    ref = _rnd(h @ W.double().T, dtype)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_err(out, ref) < tol
    ref2 = _rnd(_rnd(out.double() @ W.double().T, dtype) + emb[tok].double(), dtype)
    assert rel_err(res, ref2) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 2, 16])
def test_down_projection_release_shape(B, dtype):
    """linear_down of the released model: K = 2816 (the widest K per lane), residual in place."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(100 + B)
    K, N = 2816, 1024
    h = torch.randn(B, K, device=DEV, generator=g).to(dtype)
    W = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(dtype)
    x = torch.randn(B, N, device=DEV, generator=g).to(dtype)
    x0 = x.clone()
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(h, [(W, x, N, 0)], t_buf, resid=x)
    torch.cuda.synchronize()
    ref = _rnd(_rnd(h.double() @ W.double().T, dtype) + x0.double(), dtype)
    assert rel_err(x, ref) < (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("resid", [False, True])
@pytest.mark.parametrize("B", [2, 7, 16])
@pytest.mark.parametrize("K,N", [(1024, 1000), (2816, 1024), (352, 96)])
def test_batched_gemv_per_element(B, K, N, resid):
    """Every output of the matrix-core batched GEMV (rows in place: each lane loads its own
    activation fragments, no LDS staging; K = 2816 on 8 waves of 11 k-steps) within the rounding of
    the exact sum. The products of bf16 operands are exact in fp32, so only the fp32 accumulation
    order and the roundings differ from the exact value:
        |round(acc) - S| <= 0.5 ulp + K 2^-24 sum_k |w_k h_k|,   S = sum_k w_k h_k (float64),
    and with the residual, |round(round(acc) + r) - (S + r)| <= that + 0.5 ulp of the result.
    The same rows gathered through x_rows (the LDS-staged form, another K split over the waves) are
    held to the same bound."""
    from dispatcher_hybrid import fused_step
    from helpers import ulp_bf16
    print(f"batched gemv B={B} K={K} N={N} resid={resid}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(1000 + 17 * B + K + int(resid))
    x = torch.randn(B, K, device=DEV, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    r = torch.randn(B, N, device=DEV, generator=g).to(torch.bfloat16)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    outs = []
    for rows in (None, torch.arange(B, device=DEV)):
        out = torch.full((B, N), 9.0, device=DEV, dtype=torch.bfloat16)
        fused_step.decode_gemv(x, [(W, out, N, 0)], t_buf, resid=r if resid else None, x_rows=rows)
        outs.append(out)
    torch.cuda.synchronize()
    exact = x.double() @ W.double().T
    absum = x.double().abs() @ W.double().abs().T
    bound = 0.5 * ulp_bf16(exact.float()).double() + K * 2.0 ** -24 * absum
    if resid:
        exact = exact + r.double()
    for form, out in zip(("in place", "gathered"), outs):
        b = bound + (0.5 * ulp_bf16(out.float()).double() if resid else 0.0)
        excess = ((out.double() - exact).abs() - b).max().item()
        assert excess <= 0.0, f"{form}: an output lies {excess:.3g} past its rounding bound"


@pytest.mark.parametrize("B", [2, 16])
def test_batched_gemv_norm_direct_vs_staged(B):
    """The RMSNorm prologue of the batched GEMV: rows in place (the sum of squares over each lane's
    fragments, the row's four lanes and the waves, the fragments scaled in registers) against the
    same rows gathered through x_rows (staged in LDS, normalised once): the two sums of squares run
    in different orders, so the scale may differ in its last bit and flip a rounded activation:
    at least 99% of the outputs are equal bit for bit and the rest within 1e-3 of the largest."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(77 + B)
    K, N = 1024, 3072
    x = torch.randn(B, K, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.rand(K, device=DEV, generator=g).add(0.5).to(torch.bfloat16)
    W = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    outs = []
    for rows in (None, torch.arange(B, device=DEV)):
        out = torch.empty(B, N, device=DEV, dtype=torch.bfloat16)
        fused_step.decode_gemv(x, [(W, out, N, 0)], t_buf, norm_weight=w, x_rows=rows)
        outs.append(out)
    torch.cuda.synchronize()
    d = (outs[0].float() - outs[1].float()).abs()
    assert (d == 0).double().mean().item() >= 0.99
    assert rel_err(outs[0], outs[1]) < 1e-3


@pytest.mark.parametrize("B", [1, 2, 16])
def test_lm_head_shape(B):
    """A vocabulary-sized output (N = 50257, not a multiple of the row tiling; batch 2 and 16 take
    the matrix-core kernel with a partial last 16-row tile)."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(5)
    V, K = 50257, 1024
    W = (torch.randn(V, K, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(B, K, device=DEV, generator=g).to(torch.bfloat16)
    w = torch.rand(K, device=DEV, generator=g).add(0.5).to(torch.bfloat16)
    out = torch.full((B, V), 9.0, device=DEV, dtype=torch.bfloat16)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    fused_step.decode_gemv(x, [(W, out, V, 0)], t_buf, norm_weight=w)
    torch.cuda.synchronize()
    ref = _rnd(_norm(x, w, torch.bfloat16) @ W.double().T, torch.bfloat16)
    assert rel_err(out, ref) < 1e-2


@pytest.mark.parametrize("B", [1, 3, 64])
def test_position_advance(B):
    """t_advance: each launch adds exactly one to the position (the decode step's last launch)."""
    from dispatcher_hybrid import fused_step
    g = torch.Generator(device=DEV).manual_seed(21)
    K, N = 512, 1000                   # B = 64: 128 KB of fp32 rows, past the LDS staging limit
    x = torch.randn(B, K, device=DEV, generator=g)
    W = torch.randn(N, K, device=DEV, generator=g) / K ** 0.5
    out = torch.empty(B, N, device=DEV)
    t_buf = torch.full((1,), 41, dtype=torch.long, device=DEV)
    pos = torch.full((1,), 7, dtype=torch.long, device=DEV)
    for _ in range(3):
        fused_step.decode_gemv(x, [(W, out, N, 0)], t_buf, t_advance=pos)
    torch.cuda.synchronize()
    assert int(pos.item()) == 10 and int(t_buf.item()) == 41
    assert rel_err(out, x.double() @ W.double().T) < 1e-5


@pytest.mark.parametrize("B", [2, 5, 16])
def test_ffn_fragment_order_equals_rows(B):
    """The decoder's feed-forward with its hidden row in MFMA fragment order (the SwiGLU launch writes
    h as (16, ff) chunks, the down projection reads them contiguously) gives the same bits as the row
    layout, and h itself is the row-layout h reordered; launches off the batched matrix-core path
    reject the flags."""
    from dispatcher_hybrid import fused_step as fs
    g = torch.Generator(device=DEV).manual_seed(B)
    d, ff = 1024, 2816
    dt = torch.bfloat16
    x = torch.randn(B, d, device=DEV, generator=g).to(dt)
    nw = (torch.rand(d, device=DEV, generator=g) + 0.5).to(dt)
    wg = (torch.randn(ff, d, device=DEV, generator=g) * 0.03).to(dt)
    wu = (torch.randn(ff, d, device=DEV, generator=g) * 0.03).to(dt)
    wd = (torch.randn(d, ff, device=DEV, generator=g) * 0.02).to(dt)
    res = torch.randn(B, d, device=DEV, generator=g).to(dt)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    h_rows = torch.zeros(B, ff, device=DEV, dtype=dt)
    fs.decode_gemv(x, [(wg, h_rows, ff, 0), (wu, h_rows, ff, 0)], t_buf, norm_weight=nw, swiglu=True)
    out_rows = res.clone()
    fs.decode_gemv(h_rows, [(wd, out_rows, d, 0)], t_buf, resid=out_rows)
    h_frag = torch.zeros(16, ff, device=DEV, dtype=dt)
    fs.decode_gemv(x, [(wg, h_frag, ff, 0), (wu, h_frag, ff, 0)], t_buf, norm_weight=nw, swiglu=True, frag_out=True)
    out_frag = res.clone()
    fs.decode_gemv(h_frag[:B], [(wd, out_frag, d, 0)], t_buf, resid=out_frag, frag_in=True)
    torch.cuda.synchronize()
    # element (b, n) of the fragment layout: chunk (n // 32) * 64 + (n // 8 % 4) * 16 + b, offset n % 8
    n = torch.arange(ff, device=DEV)
    for b in range(B):
        idx = ((n // 32) * 64 + (n // 8 % 4) * 16 + b) * 8 + n % 8
        assert torch.equal(h_frag.view(-1)[idx], h_rows[b])
    assert torch.equal(out_frag, out_rows)
    with pytest.raises(ValueError):                   # batch 1 runs the row kernel: no fragment order
        fs.decode_gemv(h_frag[:1], [(wd, out_frag[:1], d, 0)], t_buf, resid=out_frag[:1], frag_in=True)
    with pytest.raises(ValueError):                   # fragment-ordered outputs only from a SwiGLU launch
        fs.decode_gemv(x, [(wu, h_frag, ff, 0)], t_buf, norm_weight=nw, frag_out=True)
