"""The bf16 noise floor of the eager path at its own rounding points.

Two bf16 implementations of the model that round at exactly the same points still differ wherever
their fp32 accumulations run in a different order: a product that lands near a bf16 rounding
midpoint rounds the other way, and the one-ulp flip travels through the following layers. The
size of that difference bounds how close any bf16 implementation with its own matrix-product
kernels can come to the eager bf16 path.

``fp32_product_accumulation()`` runs the eager path with every bf16 matrix product (``F.linear``,
``torch.matmul``, ``torch.bmm``) computed as an fp32 product of the same bf16 operands, rounded
once to bf16 -- the same rounding points as the eager path (one rounding of an fp32 accumulation
per product), only the accumulation order changed (the fp32 GEMM's blocking instead of the bf16
GEMM's). Everything else -- norms, adds, activations, the level scan, softmax -- is untouched.
Comparing the eager bf16 logits with and without it measures that floor.
"""

import contextlib

import torch
import torch.nn.functional as F

_BF16 = torch.bfloat16


def _wrap_binary(fn):
    def wrapped(a, b, *args, **kwargs):
        if (isinstance(a, torch.Tensor) and isinstance(b, torch.Tensor) and a.dtype == _BF16 and b.dtype == _BF16
                and not kwargs.get("out")):
            return fn(a.float(), b.float(), *args, **kwargs).to(_BF16)
        return fn(a, b, *args, **kwargs)
    return wrapped


def _wrap_linear(fn):
    def wrapped(x, w, bias=None):
        if x.dtype == _BF16 and w.dtype == _BF16:
            y = fn(x.float(), w.float())
            if bias is not None:
                y = y.to(_BF16) + bias       # the bias add stays a bf16 add, as in the eager path
                return y
            return y.to(_BF16)
        return fn(x, w, bias)
    return wrapped


@contextlib.contextmanager
def fp32_product_accumulation():
    """Within the block, bf16 F.linear / torch.matmul / torch.bmm are computed as fp32 products of
    their bf16 operands rounded once to bf16 (see the module docstring). Not thread-safe: it
    replaces the functions module-wide for the duration."""
    saved = (F.linear, torch.matmul, torch.bmm)
    F.linear = _wrap_linear(saved[0])
    torch.matmul = _wrap_binary(saved[1])
    torch.bmm = _wrap_binary(saved[2])
    try:
        yield
    finally:
        F.linear, torch.matmul, torch.bmm = saved
