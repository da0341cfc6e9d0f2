"""Deterministic seeded weights and tiny configs shared by the golden-vector script and the tests.

Weights come from a CPU torch.Generator, so the same (config, seed, scheme) gives bit-identical
tensors in this container and on the GPU box. Keys are the reference's state-dict names
(reference dispatcher_hybrid/modeling_dispatcher.py:50-61, 137-140, 192-194, 205-208, 220-223,
271-277).

Schemes:
  "reference": N(0, 0.02) projections / embedding / gate readouts, W1s = 0, biases at their
               config init (-2 / +2 / +2), norms at 1 (reference modeling_dispatcher.py:236-247).
  "parity":    fan-in-scaled projections, W1s nonzero, gate readouts and biases with spread and
               perturbed norm weights, so every term of the mixer moves the output (a dropped
               term, a wrong lag or a transposed operand changes the logits visibly).
"""

import math

import torch

TINY_CONFIGS = {
    # head_dim 64 (the release head width), 6 levels, window 16
    "tiny_a": dict(vocab_size=256, d_model=128, num_heads=2, dim_feedforward=352, num_layers=3,
                   max_len=64, attn_layers=(2,), attn_window=16, doc_reset=True, eot_token=255),
    # head_dim 16, 4 heads
    "tiny_b": dict(vocab_size=256, d_model=64, num_heads=4, dim_feedforward=176, num_layers=3,
                   max_len=64, attn_layers=(2,), attn_window=16, doc_reset=True, eot_token=255),
}

RELEASE_CONFIG = dict(vocab_size=50257, d_model=1024, num_heads=16, dim_feedforward=2816,
                      num_layers=18, max_len=4096, attn_layers=(8, 17), attn_window=1024,
                      doc_reset=True, eot_token=50256)


def _levels(cfg):
    return int(math.log2(cfg["max_len"]))


def is_attention(cfg, i):
    return cfg["attn_window"] > 0 and (i + 1) in tuple(cfg["attn_layers"])


def mixer_state_dict(cfg, g, prefix, scheme):
    d, H, L = cfg["d_model"], cfg["num_heads"], _levels(cfg)
    gh = d
    sd = {}
    if scheme == "reference":
        std_p = 0.02
        for n in ("linear_in", "gate_hidden", "gate_hidden_src", "linear_out"):
            sd[f"{prefix}{n}.weight"] = torch.randn(d, d, generator=g) * std_p
        sd[f"{prefix}gate_hidden_src.weight"].zero_()
        for n in ("gate_out", "forget_out", "reset_out"):
            sd[f"{prefix}{n}"] = torch.randn(L, H, gh, generator=g) * 0.02
        sd[f"{prefix}gate_out_bias"] = torch.full((L, H), float(cfg.get("gate_bias_flat", -2.0)))
        sd[f"{prefix}forget_out_bias"] = torch.full((L, H), float(cfg.get("gate_fbias_flat", 2.0)))
        sd[f"{prefix}reset_out_bias"] = torch.full((L, H), 2.0)
    else:
        std_p = 1.0 / math.sqrt(d)
        sd[f"{prefix}linear_in.weight"] = torch.randn(d, d, generator=g) * std_p
        sd[f"{prefix}gate_hidden.weight"] = torch.randn(d, d, generator=g) * std_p
        sd[f"{prefix}gate_hidden_src.weight"] = torch.randn(d, d, generator=g) * std_p
        sd[f"{prefix}linear_out.weight"] = torch.randn(d, d, generator=g) * std_p
        for n in ("gate_out", "forget_out", "reset_out"):
            sd[f"{prefix}{n}"] = torch.randn(L, H, gh, generator=g) * (1.5 / math.sqrt(gh))
        sd[f"{prefix}gate_out_bias"] = torch.randn(L, H, generator=g) * 0.5 - 0.5
        sd[f"{prefix}forget_out_bias"] = torch.randn(L, H, generator=g) * 0.5 + 1.0
        sd[f"{prefix}reset_out_bias"] = torch.randn(L, H, generator=g) * 0.5 + 1.0
    return sd


def make_state_dict(cfg, seed, scheme="parity", dtype=torch.float32):
    """Full-model state dict (tied head: lm_head.weight is embedding.weight)."""
    g = torch.Generator().manual_seed(seed)
    d, ff, V = cfg["d_model"], cfg["dim_feedforward"], cfg["vocab_size"]
    ref = scheme == "reference"
    sd = {"embedding.weight": torch.randn(V, d, generator=g) * (0.02 if ref else 0.5)}
    std_d = 0.02 if ref else 1.0 / math.sqrt(d)
    std_f = 0.02 if ref else 1.0 / math.sqrt(ff)
    for i in range(cfg["num_layers"]):
        p = f"blocks.{i}."
        if is_attention(cfg, i):
            for n in ("linear_q", "linear_k", "linear_v", "linear_out"):
                sd[f"{p}attn.{n}.weight"] = torch.randn(d, d, generator=g) * std_d
        else:
            sd.update(mixer_state_dict(cfg, g, p + "mixer.", scheme))
        sd[f"{p}ffn.linear_gate.weight"] = torch.randn(ff, d, generator=g) * std_d
        sd[f"{p}ffn.linear_up.weight"] = torch.randn(ff, d, generator=g) * std_d
        sd[f"{p}ffn.linear_down.weight"] = torch.randn(d, ff, generator=g) * std_f
        for n in ("norm1", "norm2"):
            sd[f"{p}{n}.weight"] = torch.ones(d) if ref else 1.0 + 0.1 * torch.randn(d, generator=g)
    sd["norm_out.weight"] = torch.ones(d) if ref else 1.0 + 0.1 * torch.randn(d, generator=g)
    sd["lm_head.weight"] = sd["embedding.weight"]
    return {k: v.to(dtype) for k, v in sd.items()}


def checksum(sd):
    """Order-independent float64 checksum of a state dict (detects generator drift)."""
    return float(sum(v.double().abs().sum().item() for _, v in sorted(sd.items())))


def load_into(model, sd):
    """Copy a state dict into a model (cast to the model's dtype)."""
    dt = next(model.parameters()).dtype
    missing, unexpected = model.load_state_dict({k: v.to(dt) for k, v in sd.items()}, strict=False)
    missing = [m for m in missing if m != "lm_head.weight"]
    if missing or unexpected:
        raise KeyError(f"state dict mismatch: missing {missing}, unexpected {unexpected}")
    model.tie_weights()
    return model
