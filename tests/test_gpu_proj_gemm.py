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
    # M, K, segment widths (bf16 tile form in the comment; fp32 takes the register-staged kernel)
    (1, 64, [64]),
    (130, 128, [128, 128, 128]),          # ragged M, three segments
    (1000, 256, [64, 192, 128]),          # segments that straddle the column tiles
    (1024, 1024, [1024, 1024, 1024]),     # the C2 layer (T = 1024): 64 x 64 tiles (768)
    (2048, 1024, [1024, 1024, 1024]),     # 64 x 128 tiles
    (2000, 512, [1000, 1024, 1048]),      # 64 x 128 tiles, ragged rows, segments straddling tiles
    (4096, 1024, [1024]),                 # 128 x 64 tiles (an out-projection)
    (1600, 1024, [2048]),                 # 128 x 128 tiles
    (257, 1024, [1024]),
    # at most 256 / 512 tiles of 64 x 64 keep three / two K tiles in flight (four / three LDS stages)
    (1024, 1024, [1024]),                 # the C2 out-projection: 256 tiles, four stages
    (1024, 2816, [1024]),                 # the C2 down projection: four stages, 44 K tiles
    (2048, 1024, [1024]),                 # 512 tiles, three stages
    (1500, 192, [1000]),                  # three stages, three K tiles, ragged rows and columns
    # bf16 launches with >= 160 output tiles of 256 x 256 take the persistent 8-wave kernel:
    (4096, 1024, [1024, 1024, 1024]),     # the released mixer (d = gh = 1024) at 4096 rows
    (3840, 1024, [1024, 1024, 1024]),     # the C3 decoder prefill
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
    the 64 x 128, 128 x 64 and 64 x 64 tile forms (two, three or four LDS stages) picked for fewer
    rows form the same sums in the same k order, so the first rows of a 9000-row launch equal those
    of shorter launches bit for bit."""
    from dispatcher_hybrid.fused_gates import fused_projections
    g = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn(9000, 1024, device=DEV, generator=g).to(torch.bfloat16)
    Ws = [(torch.randn(1024, 1024, device=DEV, generator=g) / 32).to(torch.bfloat16) for _ in range(3)]
    full = fused_projections(x, Ws)
    for M in (4096, 3840, 2048, 1024, 100, 1):
        part = fused_projections(x[:M].contiguous(), Ws)
        for o, f in zip(part, full):
            assert torch.equal(o, f[:M]), M
    # one 1024-wide segment: 128 x 64 tiles (4096 rows, two stages), 64 x 64 tiles in three stages
    # (2048) and four (1024, 100) against the 64 x 128 tiles of the 9000-row launch
    full = fused_projections(x, Ws[:1])[0]
    for M in (4096, 2048, 1024, 100):
        assert torch.equal(fused_projections(x[:M].contiguous(), Ws[:1])[0], full[:M]), M


# ---- dh_proj_gemm_swiglu: SwiGLU's gate and up GEMMs and its activation in one launch

SWIGLU_CASES = [
    # M, K, N (tile form of the 2N concatenated rows)
    (1, 64, 8),              # 64 x 64 tiles, one row, a partial feature tile
    (100, 128, 96),          # 64 x 64, ragged
    (1024, 1024, 2816),      # the C2 feed-forward (T = 1024): 128 x 64 tiles
    (1600, 1024, 1024),      # 128 x 128 tiles
    (2048, 1024, 2816),      # 256 x 256 persistent kernel
    (5000, 512, 1000),       # persistent kernel, ragged rows, N not a multiple of the tile's 128 features
    (1000, 1024, 2056),      # 64 x 128 tiles, a partial last feature tile
]


def _swiglu_ref(x, wg, wu):
    """The unfused product path: the two GEMMs as one dh_proj_gemm launch (same sums, same k order)
    and dh_silu_mul at the eager rounding points."""
    from dispatcher_hybrid.fused_gates import fused_projections, silu_mul
    g, u = fused_projections(x, [wg, wu])
    return silu_mul(g, u)


@pytest.mark.parametrize("case", SWIGLU_CASES)
def test_proj_gemm_swiglu_equals_gemms_then_silu_mul(case):
    """Bit-identical to the two GEMMs followed by dh_silu_mul, and within the bf16 rounding bound of
    a float64 silu(x Wg^T) * (x Wu^T) (reference modeling_dispatcher.py:197)."""
    from dispatcher_hybrid.fused_gates import fused_swiglu
    M, K, N = case
    print(f"proj_gemm_swiglu M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M * 7 + N)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    h = fused_swiglu(x, wg, wu)
    ref = _swiglu_ref(x, wg, wu)
    torch.cuda.synchronize()
    assert h.shape == (M, N) and h.dtype == torch.bfloat16
    assert torch.equal(h, ref)
    gd, ud = x.double() @ wg.double().T, x.double() @ wu.double().T
    exact = torch.nn.functional.silu(gd) * ud
    # four bf16 roundings (gate, up, silu, product), each 2^-8 relative, plus the fp32 sums
    bound = exact.abs() * 4 * 2.0 ** -8 + (gd.abs() + ud.abs()) * 2.0 ** -8 * (ud.abs() + gd.abs()) + 1e-3
    assert bool(((h.double() - exact).abs() <= bound).all())


def test_proj_gemm_swiglu_extreme_gates():
    """Gate outputs far below zero (rows of x scaled by 60, so some gates pass -87, where the epilogue
    takes the IEEE divide instead of the refined reciprocal for the whole tile) and rows of ordinary
    size: bit-identical to the two GEMMs followed by dh_silu_mul in both cases."""
    from dispatcher_hybrid.fused_gates import fused_swiglu
    g = torch.Generator(device=DEV).manual_seed(31)
    M, K, N = 1024, 1024, 2816
    x = torch.randn(M, K, device=DEV, generator=g)
    x[::7] *= 60.0                                  # every seventh row: |gate| up to several hundred
    x = x.to(torch.bfloat16)
    wg = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(N, K, device=DEV, generator=g) / K ** 0.5).to(torch.bfloat16)
    h = fused_swiglu(x, wg, wu)
    ref = _swiglu_ref(x, wg, wu)
    gate = x.float() @ wg.float().T
    assert float(gate.min()) < -87.0                # the divide branch is taken somewhere
    assert torch.equal(h, ref)


def test_proj_gemm_swiglu_every_bf16_gate():
    """The epilogue's SiLU over every bf16 gate value: x one-hot, W_gate's first column the 65536 bf16
    bit patterns and W_up's ones, so gate = the pattern and up = 1 exactly, and the output is
    round(silu(gate)). Equal to torch's bf16 SiLU bit for bit at every pattern (NaN where torch gives
    NaN), in tiles on the refined reciprocal and in the tiles holding gates below -87 (the divide).
    Subnormal gates are left out (the matrix cores flush them to zero), and so is -0: a sum that
    starts from +0 gives +0 for it, as the library GEMM does."""
    from dispatcher_hybrid.fused_gates import fused_swiglu
    M, K, N = 16, 64, 65536
    x = torch.zeros(M, K, device=DEV, dtype=torch.bfloat16)
    x[:, 0] = 1.0
    pat = torch.arange(N, device=DEV, dtype=torch.int32).to(torch.int16)
    wg = torch.zeros(N, K, device=DEV, dtype=torch.bfloat16)
    wg[:, 0] = pat.view(torch.bfloat16)
    wu = torch.zeros(N, K, device=DEV, dtype=torch.bfloat16)
    wu[:, 0] = 1.0
    h = fused_swiglu(x, wg, wu)[0]
    gate = pat.view(torch.bfloat16)
    ref = torch.nn.functional.silu(gate)
    bits = torch.arange(N, device=DEV)
    normal = ((bits >> 7) & 0xff) != 0                    # exponent field non-zero (or zero mantissa)
    normal |= (bits & 0x7f) == 0
    normal[0x8000] = False                               # -0: the GEMM's sum is +0
    nan_h, nan_r = torch.isnan(h), torch.isnan(ref)
    assert torch.equal(nan_h[normal], nan_r[normal])
    keep = normal & ~nan_r
    assert torch.equal(h[keep].view(torch.int16), ref[keep].view(torch.int16))


def test_proj_gemm_swiglu_rows_independent_of_tile_kernel():
    """As the plain GEMM: the first rows of a 5000-row launch (persistent kernel) equal those of
    shorter launches (128 x 64, 128 x 128 and 64 x 64 tiles) bit for bit."""
    from dispatcher_hybrid.fused_gates import fused_swiglu
    g = torch.Generator(device=DEV).manual_seed(13)
    x = torch.randn(5000, 1024, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(2816, 1024, device=DEV, generator=g) / 32).to(torch.bfloat16)
    wu = (torch.randn(2816, 1024, device=DEV, generator=g) / 32).to(torch.bfloat16)
    full = fused_swiglu(x, wg, wu)
    for M in (2048, 1024, 300, 1):
        assert torch.equal(fused_swiglu(x[:M].contiguous(), wg, wu), full[:M]), M


def test_proj_gemm_swiglu_batched_view_and_rejects():
    from dispatcher_hybrid import _hip
    from dispatcher_hybrid.fused_gates import fused_swiglu
    g = torch.Generator(device=DEV).manual_seed(17)
    x = torch.randn(2, 300, 128, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(96, 128, device=DEV, generator=g) / 12).to(torch.bfloat16)
    wu = (torch.randn(96, 128, device=DEV, generator=g) / 12).to(torch.bfloat16)
    h = fused_swiglu(x, wg, wu)
    assert h.shape == (2, 300, 96)
    assert torch.equal(h.view(600, 96), _swiglu_ref(x.view(600, 128), wg, wu))
    # a row-misaligned view of x is copied, not rejected
    buf = torch.zeros(600 * 128 + 1, device=DEV, dtype=torch.bfloat16)
    xv = buf[1:].view(600, 128)
    xv.copy_(x.view(600, 128))
    assert torch.equal(fused_swiglu(xv, wg, wu), h.view(600, 96))
    with pytest.raises(ValueError):
        fused_swiglu(x.float(), wg.float(), wu.float())                   # bf16 only
    with pytest.raises(ValueError):
        fused_swiglu(x, wg, wu[:64])                                       # gate / up shapes differ
    # the C-ABI's own checks: N a multiple of 8, fp32 refused
    null = _hip.ptr(h)
    assert _hip.lib.dh_proj_gemm_swiglu(_hip.DH_BF16, _hip.ptr(x), 128, 600, 128, _hip.ptr(wg), _hip.ptr(wu), 12,
                                        null, 96, _hip.stream_handle(x.device)) != 0
    assert _hip.lib.dh_proj_gemm_swiglu(_hip.DH_F32, _hip.ptr(x), 128, 600, 128, _hip.ptr(wg), _hip.ptr(wu), 96,
                                        null, 96, _hip.stream_handle(x.device)) != 0
