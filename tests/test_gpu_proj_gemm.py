"""dh_proj_gemm (the mixer's three input projections as one MFMA GEMM) against a float64 matmul
of the same operands (reference dispatcher_hybrid/modeling_dispatcher.py:63-74 computes them as
three nn.Linear calls). Bars: fp32 1e-5 relative (accumulation order only); bf16 one output
rounding (2^-8 relative to each element's magnitude) plus fp32 accumulation order."""

import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # M, K, segment widths
    (1, 64, [64]),
    (130, 128, [128, 128, 128]),          # ragged M, three segments
    (1000, 256, [64, 192, 128]),          # segments that straddle the 128-column tiles
    (4096, 1024, [1024, 1024, 1024]),     # the released mixer (d = gh = 1024): 128 x 128 tiles
    (3840, 1024, [1024, 1024, 1024]),     # the C3 decoder prefill: 128 x 128 tiles from two per CU
    (2048, 1024, [1024, 1024, 1024]),     # 64 x 128 tiles
    (2000, 512, [1000, 1024, 1048]),      # 64 x 128 tiles, ragged rows, segments straddling tiles
    (1024, 1024, [1024, 1024, 1024]),     # the C2 layer (T = 1024): 64 x 64 tiles
    (257, 1024, [1024]),
    # bf16 launches with >= 256 output tiles of 256 x 256 take the persistent 8-wave kernel:
    (6000, 1024, [1000, 1024, 1048]),     # ragged rows, segments straddling its 256-column tiles
    (9000, 512, [3000]),                  # one segment, width not a multiple of 256
    (32768, 1024, [1024, 1024, 1024]),    # the C5 layer: b = 8, T = 4096 rows
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_proj_gemm_matches_matmul(case, dtype):
    from dispatcher_hybrid.fused_gates import fused_projections
    M, K, Ns = case
    print(f"proj_gemm M={M} K={K} N={Ns} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M + K)
    x = torch.randn(M, K, device=DEV, generator=g).to(dtype)
    Ws = [(torch.randn(n, K, device=DEV, generator=g) / K ** 0.5).to(dtype) for n in Ns]
    outs = fused_projections(x, Ws)
    torch.cuda.synchronize()
    for o, w in zip(outs, Ws):
        ref = x.double() @ w.double().T
        assert o.shape == (M, w.shape[0]) and o.dtype == dtype
        if dtype == torch.float32:
            assert rel_err(o, ref) < 1e-5
        else:
            err = (o.double() - ref).abs()
            assert bool((err <= ref.abs() * 2.0 ** -8 + 2e-3).all()), err.max().item()


def test_proj_gemm_batched_view_and_rejects():
    from dispatcher_hybrid.fused_gates import fused_projections
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(2, 300, 128, device=DEV, generator=g)
    W = torch.randn(96, 128, device=DEV, generator=g)
    (o,) = fused_projections(x, [W])
    torch.cuda.synchronize()
    assert o.shape == (2, 300, 96)
    assert rel_err(o, x.double() @ W.double().T) < 1e-5
    with pytest.raises(ValueError):
        fused_projections(torch.zeros(4, 100, device=DEV), [torch.zeros(8, 100, device=DEV)])   # K % 32
    with pytest.raises(ValueError):
        fused_projections(x, [torch.zeros(6, 128, device=DEV)])                                  # N % 4


def test_proj_gemm_rows_independent_of_tile_kernel():
    """A row's outputs do not depend on the launch's row count: the 256 x 256 persistent kernel and
    the 128 x 128, 64 x 128 and 64 x 64 tile forms picked for fewer rows form the same sums in the
    same k order, so the first rows of a 9000-row launch equal those of shorter launches bit for bit."""
    from dispatcher_hybrid.fused_gates import fused_projections
    g = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn(9000, 1024, device=DEV, generator=g).to(torch.bfloat16)
    Ws = [(torch.randn(1024, 1024, device=DEV, generator=g) / 32).to(torch.bfloat16) for _ in range(3)]
    full = fused_projections(x, Ws)
    for M in (4096, 3840, 2048, 1024, 100, 1):
        part = fused_projections(x[:M].contiguous(), Ws)
        for o, f in zip(part, full):
            assert torch.equal(o, f[:M]), M
