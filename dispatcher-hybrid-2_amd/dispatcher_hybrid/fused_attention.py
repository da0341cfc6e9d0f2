"""Banded causal attention of a whole sequence on gfx950 (``dh_window_attention_fwd``).

Used by WindowAttention.forward under ``model.enable_fused_gates()`` for inference (no autograd)
and by the fused decoder's prefill, which also has the kernel write the rotated keys and the
values into the decoder caches (reference dispatcher_hybrid/modeling_dispatcher.py:168-182,
dispatcher_hybrid/decoding.py:143-185). bf16 and head widths 32 / 64 / 128; other cases stay on the
torch path of the caller. Importing this module loads the kernel library (ImportError if missing).
"""

import torch

from . import _hip

HEAD_DIMS = (32, 64, 128)


def supported(dtype, head_dim):
    """Whether the kernel takes this dtype / head width."""
    return dtype == torch.bfloat16 and head_dim in HEAD_DIMS


def window_attention(q, k, v, rope_cos, rope_sin, num_heads, window, k_cache=None, v_cache=None):
    """y = softmax(rope(q) rope(k)^T / sqrt(hd)) v over keys s with t - window < s <= t (window 0:
    all s <= t), per head. q, k, v: (B, T, H*hd) projections before RoPE with identical strides and
    a unit inner stride. rope_cos / rope_sin: (>= T, hd/2). Returns y (B, T, H*hd). k_cache /
    v_cache: optional (B, H, Tmax, hd) decoder caches whose rows [0, T) receive rope(k) and v."""
    for x in (q, k, v):
        _hip.require_gpu(x, "window_attention")
    B, T, d = q.shape
    hd = d // num_heads
    if not supported(q.dtype, hd):
        raise TypeError(f"window_attention: bf16 with head width in {HEAD_DIMS} only (got {q.dtype}, hd {hd})")
    if k.shape != q.shape or v.shape != q.shape or not (q.stride() == k.stride() == v.stride()) or q.stride(-1) != 1:
        raise ValueError("window_attention: q, k, v must have one shape and one stride, unit inner stride")
    if k.dtype != q.dtype or v.dtype != q.dtype or rope_cos.dtype != q.dtype or rope_sin.dtype != q.dtype:
        raise TypeError("window_attention: q, k, v and the rope tables must share one dtype")
    if rope_cos.shape[0] < T or rope_cos.shape[-1] != hd // 2 or not rope_cos.is_contiguous() or not rope_sin.is_contiguous():
        raise ValueError("window_attention: rope tables must be contiguous (>= T, hd/2)")
    y = torch.empty(B, T, d, device=q.device, dtype=q.dtype)
    if (k_cache is None) != (v_cache is None):
        raise ValueError("window_attention: give both caches or neither")
    if k_cache is None:      # the kernel stages rope(k) and v head-major: scratch for the forward
        k_cache = torch.empty(B, num_heads, T, hd, device=q.device, dtype=q.dtype)
        v_cache = torch.empty_like(k_cache)
    else:
        if (k_cache.shape != v_cache.shape or k_cache.dtype != q.dtype or k_cache.shape[0] != B or
                k_cache.shape[1] != num_heads or k_cache.shape[3] != hd or k_cache.stride(-1) != 1 or
                k_cache.stride(2) != hd or k_cache.stride() != v_cache.stride()):
            raise ValueError("window_attention: caches must be (B, H, Tmax, hd) with rows of hd elements")
    Tmax, cb, ch = k_cache.shape[2], k_cache.stride(0), k_cache.stride(1)
    p = _hip.ptr
    st = _hip.lib.dh_window_attention_fwd(
        _hip.dtype_code(q.dtype), p(q), p(k), p(v), q.stride(0), q.stride(1), p(rope_cos), p(rope_sin),
        p(y), y.stride(0), y.stride(1), p(k_cache), p(v_cache), cb, ch, Tmax, B, T, num_heads, hd,
        int(window), _hip.stream_handle(q.device))
    _hip.check(st, "dh_window_attention_fwd")
    return y
