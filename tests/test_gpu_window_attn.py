"""dh_window_attention_fwd (banded causal attention with RoPE, the forward and decoder prefill of
an attention layer) against float64 attention over the same rotated bf16 queries and keys, the
product's eager bf16 attention, and the eager prefill's cache rows (reference
dispatcher_hybrid/modeling_dispatcher.py:163-182, dispatcher_hybrid/decoding.py:143-185)."""

import math

import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
DT = torch.bfloat16


def _rope_tables(T, hd):
    inv = torch.pow(10000.0, -torch.arange(0, hd, 2, device=DEV, dtype=torch.float32) / hd)
    ang = torch.outer(torch.arange(T, device=DEV, dtype=torch.float32), inv)
    return ang.cos().to(DT), ang.sin().to(DT)


def _inputs(B, T, H, hd, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    mk = lambda: torch.randn(B, T, H * hd, device=DEV, generator=g).to(DT)
    return mk(), mk(), mk()


def _rotated(x, cos, sin, H):
    """The eager bf16 rope of (B, T, H*hd) rows: (B, T, H, hd)."""
    from dispatcher_hybrid.modeling_dispatcher import rope_rotate
    B, T, d = x.shape
    return rope_rotate(x.view(B, T, H, d // H), cos[:T].unsqueeze(1), sin[:T].unsqueeze(1))


def _reference(q, k, v, cos, sin, H, window):
    """float64 banded attention over the bf16-rotated queries and keys: (B, T, H*hd)."""
    B, T, d = q.shape
    hd = d // H
    qr, kr = _rotated(q, cos, sin, H).double(), _rotated(k, cos, sin, H).double()
    vv = v.view(B, T, H, hd).double()
    s = torch.einsum("bthd,bshd->bhts", qr, kr) / math.sqrt(hd)
    t = torch.arange(T, device=DEV)
    ok = t[:, None] >= t[None, :]
    if window > 0:
        ok = ok & (t[:, None] - t[None, :] < window)
    p = torch.softmax(s.masked_fill(~ok, float("-inf")), dim=-1)
    return torch.einsum("bhts,bshd->bthd", p, vv).reshape(B, T, d)


# (B, T, H, hd, window): a single position, ragged blocks, windows inside / at / beyond one 64-key
# block, every head width, the released shape (window 1024 of 4096)
CASES = [(1, 1, 2, 64, 0), (2, 37, 3, 64, 0), (1, 200, 2, 32, 16), (2, 300, 2, 128, 100),
         (3, 130, 2, 64, 64), (1, 1024, 4, 64, 0), (1, 1500, 2, 64, 1024), (1, 4096, 2, 64, 1024)]


@pytest.mark.parametrize("case", CASES)
def test_window_attention_matches_float64(case):
    from dispatcher_hybrid import fused_attention as fa
    from dispatcher_hybrid.modeling_dispatcher import causal_window_attention
    B, T, H, hd, window = case
    print(f"window attention case={case}", flush=True)
    q, k, v = _inputs(B, T, H, hd, T + hd)
    cos, sin = _rope_tables(T, hd)
    y = fa.window_attention(q, k, v, cos, sin, H, window)
    torch.cuda.synchronize()
    ref = _reference(q, k, v, cos, sin, H, window)
    err = rel_err(y, ref)
    # the eager bf16 path of the product on the same inputs: the kernel must be no further from float64
    qe = _rotated(q, cos, sin, H).transpose(1, 2)
    ke = _rotated(k, cos, sin, H).transpose(1, 2)
    ye = causal_window_attention(qe, ke, v.view(B, T, H, hd).transpose(1, 2), window)
    eager_err = rel_err(ye.transpose(1, 2).reshape(B, T, H * hd), ref)
    assert err < 1.5e-2, f"rel {err:.3e}"
    assert err <= 1.5 * eager_err + 1e-3, f"kernel {err:.3e} vs eager {eager_err:.3e}"


@pytest.mark.parametrize("T,window", [(37, 0), (200, 64), (131, 16)])
def test_window_attention_cache_rows_bit_exact(T, window):
    """With caches the kernel writes rope(k) and v into rows [0, T) of (B, H, Tmax, hd): equal bit
    for bit to the eager bf16 rope and the raw values; rows from T on stay untouched."""
    from dispatcher_hybrid import fused_attention as fa
    B, H, hd, Tmax = 2, 2, 64, 256
    q, k, v = _inputs(B, T, H, hd, 7 * T)
    cos, sin = _rope_tables(Tmax, hd)
    kc = torch.full((B, H, Tmax, hd), 3.0, device=DEV, dtype=DT)
    vc = torch.full((B, H, Tmax, hd), 3.0, device=DEV, dtype=DT)
    fa.window_attention(q, k, v, cos, sin, H, window, k_cache=kc, v_cache=vc)
    torch.cuda.synchronize()
    assert torch.equal(kc[:, :, :T], _rotated(k, cos, sin, H).transpose(1, 2))
    assert torch.equal(vc[:, :, :T], v.view(B, T, H, hd).transpose(1, 2))
    assert bool((kc[:, :, T:] == 3.0).all()) and bool((vc[:, :, T:] == 3.0).all())


def test_window_attention_rejects_unsupported():
    from dispatcher_hybrid import fused_attention as fa
    q, k, v = _inputs(1, 8, 2, 64, 1)
    cos, sin = _rope_tables(8, 64)
    with pytest.raises(TypeError, match="bf16"):
        fa.window_attention(q.float(), k.float(), v.float(), cos.float(), sin.float(), 2, 0)
    with pytest.raises(TypeError, match="head width"):
        fa.window_attention(q, k, v, cos, sin, 8, 0)                 # hd 16
    k_wide = torch.empty(1, 8, 256, device=DEV, dtype=DT)[..., :128]           # rows 256 apart
    k_wide.copy_(k)
    with pytest.raises(ValueError, match="one stride"):
        fa.window_attention(q, k_wide, v, cos, sin, 2, 0)
