"""Empty inputs through the fused parallel path: no launch, outputs of the right shapes.

The eager mixer (reference dispatcher_hybrid/modeling_dispatcher.py:86-121) runs on an empty
batch or a zero-length sequence as any torch op does; the fused ops (same signatures as reference
dispatcher_hybrid/fused_gates.py:307-314) must give the same shapes, and their autograd backward
zero-sized gradients, without launching a kernel on an empty grid.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("b,T", [(2, 0), (0, 5), (0, 0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_empty_gate_path(b, T, dtype):
    from dispatcher_hybrid import fused_gates
    print(f"empty gate path b={b} T={T} {dtype}", flush=True)
    L, H, GH, hd, n_lv = 4, 2, 64, 16, 3
    g = torch.Generator(device=DEV).manual_seed(1)
    A = torch.randn(b, T, GH, device=DEV, generator=g).to(dtype).requires_grad_()
    B = torch.randn(b, T, GH, device=DEV, generator=g).to(dtype).requires_grad_()
    Ws = [(torch.randn(L, H, GH, device=DEV, generator=g) * 0.1).to(dtype).requires_grad_() for _ in range(3)]
    bs = [torch.zeros(L, H, device=DEV, dtype=dtype, requires_grad=True) for _ in range(3)]
    pre = fused_gates.fused_gate_preacts(A, B, *Ws, *bs, n_lv)
    for p in pre:
        assert p.shape == (b, T, n_lv, H)
    sum(p.float().sum() for p in pre).backward()
    assert A.grad.shape == A.shape and B.grad.shape == B.shape
    for w in Ws:
        assert w.grad.shape == w.shape and bool((w.grad == 0).all())
    for v in bs:
        assert v.grad.shape == v.shape and bool((v.grad == 0).all())

    V0 = torch.randn(b, T, H * hd, device=DEV, generator=g).to(dtype)
    with torch.no_grad():
        Y = fused_gates.fused_level_scan(*[p.detach() for p in pre], None, V0, H, n_lv)
        Z = fused_gates.fused_gate_scan(A.detach(), B.detach(), *[w.detach() for w in Ws],
                                        *[v.detach() for v in bs], n_lv, None, V0, H)
    torch.cuda.synchronize()
    assert Y.shape == V0.shape and Z.shape == V0.shape
    assert Y.dtype == V0.dtype and Z.dtype == V0.dtype
