"""Shared test helpers: golden fixtures, seeded models, comparison metrics."""

import os

import numpy as np
import torch

from weights import TINY_CONFIGS, checksum, load_into, make_state_dict

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEED_WEIGHTS = 1234


def golden(name):
    return dict(np.load(os.path.join(GOLDEN, f"{name}.npz")))


def config(cfgd):
    from dispatcher_hybrid import DispatcherConfig
    return DispatcherConfig(**cfgd)


def product_model(cfgd, sd, device="cpu", dtype=torch.float32):
    from dispatcher_hybrid import DispatcherHybridForCausalLM
    with torch.device(device):                       # initialise in place (fast on the GPU)
        m = DispatcherHybridForCausalLM(config(cfgd)).eval()
    m = m.to(dtype=dtype)
    load_into(m, sd)
    return m


def tiny(name, scheme="parity", seed=SEED_WEIGHTS):
    cfgd = TINY_CONFIGS[name]
    sd = make_state_dict(cfgd, seed, scheme=scheme)
    return cfgd, sd


def rel_err(got, ref):
    got = torch.as_tensor(got).double()
    ref = torch.as_tensor(ref).double()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def max_abs(got, ref):
    return (torch.as_tensor(got).double() - torch.as_tensor(ref).double()).abs().max().item()


def argmax_agree(got, ref):
    return (torch.as_tensor(got).argmax(-1) == torch.as_tensor(ref).argmax(-1)).double().mean().item()


def decisive_argmax_agree(got, ref, margin=0.75):
    """argmax must agree wherever the reference's top-2 margin exceeds `margin`
    (the reference's own bf16 criterion, reference tests/test_decoding.py:61-68)."""
    ref = torch.as_tensor(ref).float()
    got = torch.as_tensor(got).float()
    top2 = torch.topk(ref, 2, dim=-1).values
    decisive = (top2[..., 0] - top2[..., 1]) > margin
    agree = got.argmax(-1) == ref.argmax(-1)
    return bool((agree | ~decisive).all())


def bf16_round(x):
    return torch.as_tensor(x).to(torch.bfloat16).to(torch.float64)
