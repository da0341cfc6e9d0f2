"""dh_argmax_noalloc, the entry point that allocates nothing (no counterpart in the reference; for
callers that cannot allocate device memory), against dh_argmax with a caller workspace, called
through the C-ABI: two calls in a row, the second on a smaller input, each equal to dh_argmax's
result and to torch.argmax (ties: first index; NaN above every number); inputs beyond the fixed
scratch are rejected before any launch."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib():
    from dispatcher_hybrid import _hip
    return _hip


def _argmax_ws(h, logits):
    B, V = logits.shape
    nbytes = int(h.lib.dh_argmax_workspace_bytes(B, V))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    out = torch.full((B,), -1, dtype=torch.long, device=DEV)
    st = h.lib.dh_argmax(h.dtype_code(logits.dtype), h.ptr(logits), logits.stride(0), B, V, h.ptr(out), h.ptr(ws),
                         nbytes, h.stream_handle(logits.device))
    assert st == 0, h.lib.dh_last_error()
    return out


def _argmax_noalloc(h, logits):
    B, V = logits.shape
    out = torch.full((B,), -1, dtype=torch.long, device=DEV)
    st = h.lib.dh_argmax_noalloc(h.dtype_code(logits.dtype), h.ptr(logits), logits.stride(0), B, V, h.ptr(out),
                                 h.stream_handle(logits.device))
    assert st == 0, h.lib.dh_last_error()
    return out


def _logits(B, V, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(B, V, device=DEV, generator=g).to(dtype)
    x[0, V // 3] = x[0, V // 5] = 40.0                      # tie: the first index wins
    if B > 2:
        x[2, V - 1] = float("nan")                          # NaN above every number
        x[2, 7] = float("nan")                              # ... the first NaN
    return x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_argmax_equals_workspace_argmax_twice(dtype):
    h = _lib()
    for B, V, seed in ((16, 50257, 1), (3, 3001, 2)):        # the second call smaller
        print(f"no-alloc argmax B={B} V={V} {dtype}", flush=True)
        x = _logits(B, V, dtype, seed)
        got = _argmax_noalloc(h, x)
        ref = _argmax_ws(h, x)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        assert torch.equal(got, x.argmax(-1))


def test_noalloc_argmax_wrapper_and_limit():
    from dispatcher_hybrid import fused_step
    h = _lib()
    x = _logits(4, 1000, torch.float32, 3)
    out = torch.empty(4, dtype=torch.long, device=DEV)
    assert torch.equal(fused_step.argmax_tokens_noalloc(x, out), x.argmax(-1))
    big = torch.zeros(400, 50257, dtype=torch.bfloat16, device=DEV)   # 400 * 25 candidates > 8192
    st = h.lib.dh_argmax_noalloc(h.dtype_code(big.dtype), h.ptr(big), big.stride(0), 400, 50257,
                                 h.ptr(torch.empty(400, dtype=torch.long, device=DEV)), h.stream_handle(big.device))
    assert st == 2 and b"fixed scratch" in h.lib.dh_last_error()
    with pytest.raises(Exception, match="fixed scratch"):
        fused_step.argmax_tokens_noalloc(big, torch.empty(400, dtype=torch.long, device=DEV))
