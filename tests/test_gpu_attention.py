"""dh_decode_attention (one windowed RoPE attention decode step in one launch) against the eager
step restated in float64 with the eager bf16 rounding points (reference
dispatcher_hybrid/decoding.py:247-266 eager step, :411-435 graph step; modeling_dispatcher.py:163-166).

Bars: fp32 within 1e-5 relative; bf16 within 1e-2 relative (probabilities and the value average
rounded at the same points, accumulation order differs); the cache row written at t bit-exact
against torch's own bf16 RoPE ops."""

import math

import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rope_tables(Tmax, hd, dtype):
    inv = torch.pow(10000.0, -torch.arange(0, hd, 2, device=DEV, dtype=torch.float32) / hd)
    ang = torch.outer(torch.arange(Tmax, device=DEV, dtype=torch.float32), inv)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def _rope_torch(x, cos, sin):
    """torch ops in x's dtype, as the eager decoder rotates (interleaved pairs)."""
    pairs = x.unflatten(-1, (-1, 2))
    even, odd = pairs[..., 0], pairs[..., 1]
    return torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(-2)


def _reference(q, k, v, cos, sin, K, V, t, window, dtype):
    """float64 restatement of the eager step; rnd() applies the bf16 rounding points."""
    rnd = (lambda x: x.to(dtype).double()) if dtype == torch.bfloat16 else (lambda x: x)
    B, H, Tmax, hd = K.shape
    qr = _rope_torch(q.view(B, H, hd), cos[t], sin[t]).double()
    kr = _rope_torch(k.view(B, H, hd), cos[t], sin[t])
    Kc, Vc = K.double().clone(), V.double().clone()
    Kc[:, :, t] = kr.double()
    Vc[:, :, t] = v.view(B, H, hd).double()
    lo = max(0, t + 1 - window) if window > 0 else 0
    s = torch.einsum("bhd,bhjd->bhj", qr, Kc[:, :, lo:t + 1])
    s = rnd(rnd(s) / math.sqrt(hd))
    p = rnd(torch.softmax(s, dim=-1))
    y = torch.einsum("bhj,bhjd->bhd", p, Vc[:, :, lo:t + 1])
    return rnd(y).reshape(B, H * hd), kr


CASES = [
    # B, H, hd, Tmax, window, t
    (1, 16, 64, 4096, 1024, 4000),        # released shape, window full
    (2, 4, 16, 64, 16, 5),                # window not yet full, hd 16
    (3, 2, 32, 100, 0, 99),               # whole prefix (window 0)
    (1, 2, 128, 300, 256, 0),             # first position, hd 128
    (16, 16, 64, 4096, 1024, 1500),       # batch 16
    (1, 1, 64, 2048, 0, 2047),            # 2048 positions: more than one sweep per thread
    (1, 16, 64, 4096, 0, 4095),           # whole prefix: 256 positions per split segment (2 sweeps)
    (2, 3, 128, 40, 0, 3),                # fewer positions than segments (empty segments)
]


@pytest.mark.parametrize("split", [False, True], ids=["one_launch", "split_window"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_decode_attention_matches_eager_step(case, dtype, split):
    """split_window (dh_decode_attention_split) keeps the probabilities in fp32 where the eager bf16
    step rounds them: its bf16 bar is the same 1e-2 relative (the rounding moves y by ~2^-9 of the
    value average's magnitude)."""
    from dispatcher_hybrid import fused_step
    B, H, hd, Tmax, window, t = case
    print(f"decode_attention case={case} {dtype} split={split}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(hd * 31 + t)
    d = H * hd
    q = torch.randn(B, d, device=DEV, generator=g).to(dtype)
    k = torch.randn(B, d, device=DEV, generator=g).to(dtype)
    v = torch.randn(B, d, device=DEV, generator=g).to(dtype)
    K = torch.randn(B, H, Tmax, hd, device=DEV, generator=g).to(dtype)
    V = torch.randn(B, H, Tmax, hd, device=DEV, generator=g).to(dtype)
    cos, sin = _rope_tables(Tmax, hd, dtype)
    ref_y, ref_k = _reference(q, k, v, cos, sin, K, V, t, window, dtype)
    K0, V0 = K.clone(), V.clone()
    y = torch.full((B, d), 7.0, device=DEV, dtype=dtype)
    t_buf = torch.full((1,), t, dtype=torch.long, device=DEV)
    ws = fused_step.attention_workspace(B, H, hd, DEV) if split else None
    if ws is not None:
        ws.fill_(float("nan"))                           # every record read is written first
    fused_step.decode_attention(q, k, v, cos, sin, K, V, t_buf, y, window, workspace=ws)
    torch.cuda.synchronize()
    assert rel_err(y, ref_y) < (1e-5 if dtype == torch.float32 else 1e-2)
    # the cache changes in row t only: the rotated key and the value, bit for bit
    assert torch.equal(K[:, :, t], ref_k)
    assert torch.equal(V[:, :, t], v.view(B, H, hd))
    rest = torch.ones(Tmax, dtype=torch.bool, device=DEV)
    rest[t] = False
    assert torch.equal(K[:, :, rest], K0[:, :, rest]) and torch.equal(V[:, :, rest], V0[:, :, rest])


@pytest.mark.parametrize("split", [False, True], ids=["one_launch", "split_window"])
def test_decode_attention_position_out_of_range_writes_nothing(split):
    from dispatcher_hybrid import fused_step
    B, H, hd, Tmax = 1, 2, 64, 32
    q = torch.randn(B, H * hd, device=DEV)
    K = torch.randn(B, H, Tmax, hd, device=DEV)
    V = torch.randn_like(K)
    K0, V0 = K.clone(), V.clone()
    cos, sin = _rope_tables(Tmax, hd, torch.float32)
    y = torch.full((B, H * hd), 3.0, device=DEV)
    t_buf = torch.full((1,), Tmax, dtype=torch.long, device=DEV)
    ws = fused_step.attention_workspace(B, H, hd, DEV) if split else None
    fused_step.decode_attention(q, q, q, cos, sin, K, V, t_buf, y, 0, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(K, K0) and torch.equal(V, V0) and bool((y == 3.0).all())


def test_decode_attention_rejects_bad_arguments():
    from dispatcher_hybrid import fused_step
    K = torch.zeros(1, 2, 16, 48, device=DEV)
    x = torch.zeros(1, 96, device=DEV)
    cos = torch.zeros(16, 24, device=DEV)
    t_buf = torch.zeros(1, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="hd=48"):
        fused_step.decode_attention(x, x, x, cos, cos, K, K.clone(), t_buf, x.clone(), 0)
    with pytest.raises(TypeError):
        fused_step.decode_attention(x.bfloat16(), x, x, cos, cos, K, K.clone(), t_buf, x.clone(), 0)
