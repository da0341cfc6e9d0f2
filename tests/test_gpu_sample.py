"""dh_argmax (greedy next token on the device) against torch.argmax, the call it replaces in
fast_generate's greedy branch (reference dispatcher_hybrid/modeling_dispatcher.py:426-441):
same index bit for bit, including ties (first index) and NaN (first NaN)."""

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
