"""Write the golden vectors under tests/golden/ from the REFERENCE's own CPU eager paths.

    python tests/golden/make_golden.py        (in the build container only: needs /root/reference)

The reference package (/root/reference/dispatcher_hybrid) is imported here, and only here, to pin
the functions no closed form or invariant pins on its own: the end-to-end forward composition
(RMSNorm eps, interleaved RoPE, banded SDPA, tied head), the doc-reset tree mask, the eager
incremental decoder's state (including beyond-horizon transmit gates and ring slabs) and greedy
fast_generate. Weights and inputs come from seeded CPU generators (tests/golden/weights.py), so only
outputs are stored. Nothing from the reference is stored but these input/output vectors.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = os.environ.get("DISPATCHER_REFERENCE", "/root/reference")
sys.path.insert(0, HERE)
sys.path.insert(0, REFERENCE)

from weights import (RELEASE_CONFIG, TINY_CONFIGS, checksum, load_into,  # noqa: E402
                     make_state_dict, mixer_state_dict)

SEED_WEIGHTS = 1234
SEED_INPUTS = 7


def f32(t):
    return t.detach().float().numpy()


def main():
    from dispatcher_hybrid import DispatcherConfig, DispatcherHybridForCausalLM
    from dispatcher_hybrid.decoding import IncrementalDecoder
    import dispatcher_hybrid
    assert os.path.realpath(dispatcher_hybrid.__file__).startswith(os.path.realpath(REFERENCE)), \
        "must import the reference package"
    torch.set_grad_enabled(False)

    for name, cfgd in TINY_CONFIGS.items():
        sd = make_state_dict(cfgd, SEED_WEIGHTS, scheme="parity")
        model = load_into(DispatcherHybridForCausalLM(DispatcherConfig(**cfgd)).eval(), sd)
        V, eot = cfgd["vocab_size"], cfgd["eot_token"]
        g = torch.Generator().manual_seed(SEED_INPUTS)
        ids = torch.randint(0, V - 1, (2, 48), generator=g)
        ids[1, 20] = eot
        ids[0, 33] = eot
        logits = model(ids).logits
        tmask = model._tree_mask(ids, ids.shape[1])
        prompts = torch.randint(0, V - 1, (2, 32), generator=g)     # EOT-free (eot = V-1)
        nexts = torch.randint(0, V - 1, (2, 8), generator=g)
        dec = IncrementalDecoder(model)
        prefill_logits = dec.prefill(prompts)
        step_logits = torch.stack([dec.step(nexts[:, j]) for j in range(nexts.shape[1])], dim=1)
        tree0 = dec.caches[0]
        Tn = prompts.shape[1] + nexts.shape[1]
        gen = model.fast_generate(prompts[:1, :6], max_new_tokens=10, decoder="eager")
        np.savez_compressed(
            os.path.join(HERE, f"{name}.npz"),
            weights_seed=SEED_WEIGHTS, weights_checksum=checksum(sd),
            ids=ids.numpy(), logits=f32(logits), tree_mask=f32(tmask),
            prompts=prompts.numpy(), nexts=nexts.numpy(),
            prefill_logits=f32(prefill_logits), step_logits=f32(step_logits),
            B_hist0=f32(tree0.B_hist[:, :Tn]), rg_hist0=f32(tree0.rg_hist[:, :Tn]),
            V_ring0=f32(tree0.V_ring), gen=gen.numpy())
        print(name, "logits", tuple(logits.shape), "gen", gen.tolist())

    # one release-shaped mixer layer (d 1024, 16 heads, 12 levels) at T = 40
    cfgd = dict(RELEASE_CONFIG, vocab_size=256, eot_token=255, num_layers=1, attn_layers=())
    model = DispatcherHybridForCausalLM(DispatcherConfig(**cfgd)).eval()
    mixer = model.blocks[0].mixer
    g = torch.Generator().manual_seed(99)
    msd = mixer_state_dict(cfgd, g, "", "parity")
    mixer.load_state_dict(msd)
    T = 40
    x = torch.randn(1, T, cfgd["d_model"], generator=g)
    ids = torch.randint(0, 255, (1, T), generator=g)
    ids[0, 13] = 255
    ids[0, 29] = 255
    tmask = model._tree_mask(ids, T)
    captured = {}
    hook = mixer.linear_out.register_forward_hook(lambda m, inp, out: captured.__setitem__("V", inp[0]))
    y_doc = mixer(x, tmask)
    V_doc = captured["V"]
    y_level = mixer(x, model.level_mask(T, dtype=x.dtype))
    hook.remove()
    np.savez_compressed(os.path.join(HERE, "release_mixer.npz"), weights_seed=99,
                        weights_checksum=checksum(msd), ids=ids.numpy(), tree_mask=f32(tmask),
                        V_doc=f32(V_doc), y_doc=f32(y_doc), y_level=f32(y_level))
    print("release_mixer", tuple(y_doc.shape))


if __name__ == "__main__":
    main()
