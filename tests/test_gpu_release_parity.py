"""Parity at the benchmark configs' own sizes on the released 292M architecture (random init):

  C4  batch 16 after a 3840-token shared prefix, decoded to the last position t = 4095
      (reference tests/test_decoding.py:134-178: batched = solo, batched fused in bf16), and the
      captured top-k sampler (step_sample) at that shape against step() + the same sampler
  C5  one fused forward at B = 8, T = 4096 with planted document separators against the eager
      forward (reference modeling_dispatcher.py:325-359)

Batch-16 bf16 rows are not compared bit for bit with batch-1 runs of the same row: batch 1 runs
the row GEMV (each lane a K slice, DPP reductions) and the batch-1 mixer step form, batch 16 the
matrix-core batch GEMV and dh_decode_mixer_step, whose fp32 sums run in other orders; bf16 rounding
then differs by an ulp here and there. fp32 rows are held to batched = solo (rel <= 1e-4) instead,
and bf16 to the model-level bf16 criterion (helpers.bf16_vs_truth).
"""

import pytest
import torch

from dispatcher_hybrid.numerics import fp32_product_accumulation
from helpers import bf16_vs_truth, product_model, rel_err
from weights import RELEASE_CONFIG, make_state_dict

pytestmark = pytest.mark.gpu
DEV = "cuda"
PREFIX, TMAX = 3840, 4096


@pytest.fixture(scope="module")
def release():
    """292M random init (reference scheme, W1s ~ N(0, 0.02) so every lag's source row matters), fp32
    and bf16 on the GPU, and the C4 inputs: one shared 3840-token prefix for 16 rows and each row's
    own 256 continuation tokens (positions 3840 .. 4095)."""
    cfgd = RELEASE_CONFIG
    sd = make_state_dict(cfgd, 0, scheme="reference")
    g = torch.Generator().manual_seed(1)
    for k in list(sd):
        if k.endswith("gate_hidden_src.weight"):
            sd[k] = torch.randn(sd[k].shape, generator=g) * 0.02
    m32 = product_model(cfgd, sd, device=DEV)
    m16 = product_model(cfgd, sd, device=DEV, dtype=torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(40)
    V = cfgd["vocab_size"]
    prefix = torch.randint(0, V - 1, (1, PREFIX), device=DEV, generator=g).expand(16, -1).contiguous()
    nexts = torch.randint(0, V - 1, (16, TMAX - PREFIX), device=DEV, generator=g)
    return cfgd, m32, m16, prefix, nexts


def _forced(dec, prompt, toks, rows=None):
    """Logits (B, n, V) fp32 of dec after prefill(prompt), each step fed toks[:, j]; when `rows` is
    given only those rows are kept (host memory of 16 x 256 x 50257 fp32 logits is avoided)."""
    dec.prefill(prompt)
    out = []
    for j in range(toks.shape[1]):
        lg = dec.step(toks[:, j]).float()
        out.append(lg if rows is None else lg[rows])
        if j % 64 == 63:
            print(f"  {type(dec).__name__} step {j + 1}/{toks.shape[1]}", flush=True)
    return torch.stack(out, 1)


def test_c4_fp32_batched_equals_solo_to_4095(release):
    """C4 in fp32: the batch-16 fused decoder's rows 0, 7 and 15 against solo eager decoders of the
    same row, every step t = 3840 .. 4095: rel <= 1e-4 and equal argmax."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    cfgd, m32, _, prefix, nexts = release
    rows = [0, 7, 15]
    print("C4 fp32 batched fused decoder, B=16", flush=True)
    b32 = _forced(FusedGraphedHybridDecoder(m32), prefix, nexts, rows)
    for i, r in enumerate(rows):
        print(f"C4 fp32 solo eager row {r}", flush=True)
        solo = _forced(IncrementalDecoder(m32), prefix[r:r + 1], nexts[r:r + 1])[0]
        rr = rel_err(b32[i], solo)
        print(f"C4 fp32 row {r}: batched fused vs solo eager rel={rr:.2e} over t={PREFIX}..{TMAX - 1}", flush=True)
        assert rr <= 1e-4
        assert bool((b32[i].argmax(-1) == solo.argmax(-1)).all())


def test_c4_bf16_batched_to_4095(release):
    """C4 in bf16: the batch-16 fused decoder (matrix-core batch GEMVs, dh_decode_mixer_step) against
    the eager bf16 and fp32 decoders over t = 3840 .. 4095 (six of the 16 rows kept), the model-level
    bf16 criterion with the same-rounding floor measured on the same steps."""
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    cfgd, m32, m16, prefix, nexts = release
    rows = list(range(0, 16, 3))                     # 6 rows x 256 steps of logits kept per run
    print("C4 bf16 fused B=16", flush=True)
    f16 = _forced(FusedGraphedHybridDecoder(m16), prefix, nexts, rows)
    print("C4 bf16 eager B=16", flush=True)
    e16 = _forced(IncrementalDecoder(m16), prefix, nexts, rows)
    print("C4 bf16 eager B=16, fp32 product accumulation (the same-rounding floor)", flush=True)
    with fp32_product_accumulation():
        a16 = _forced(IncrementalDecoder(m16), prefix, nexts, rows)
    print("C4 fp32 eager B=16", flush=True)
    t32 = _forced(IncrementalDecoder(m32), prefix, nexts, rows)
    bf16_vs_truth(f16, e16, t32, "C4 bf16 B=16 t=3840..4095", alt16=a16)


def test_c4_step_sample_equals_step_and_sampler(release):
    """The C4 bench path: step_sample (dh_sample_topk as the captured step's last launch,
    temperature 0.8, top-k 50) at batch 16 on the bf16 release model from the 3840-token shared
    prefix to t = 4095, against a second decoder running step() and then sample_tokens with the
    same settings and the device position: the same 256 x 16 tokens, each inside its row's top-50."""
    from dispatcher_hybrid import fused_step
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    cfgd, _, m16, prefix, _ = release
    T, K, seed = 0.8, 50, 1234
    n = TMAX - PREFIX
    da = FusedGraphedHybridDecoder(m16)
    da.sample_start(da.prefill(prefix)[:, -1], temperature=T, top_k=K, seed=seed)
    for _ in range(n - 1):
        da.step_sample()
    got = da.tok_hist[:, PREFIX:PREFIX + n].clone()
    db = FusedGraphedHybridDecoder(m16)
    lg = db.prefill(prefix)[:, -1]
    tok = fused_step.sample_tokens(lg, T, K, seed, db.t_buf)
    ref, outside = [tok], 0
    for j in range(n - 1):
        lg = db.step(tok)
        tok = fused_step.sample_tokens(lg, T, K, seed, db.t_buf)
        kth = torch.topk(lg.float(), K, dim=-1).values[:, -1:]
        outside += int((lg.float().gather(1, tok[:, None]) < kth).sum())
        ref.append(tok)
    ref = torch.stack(ref, 1)
    same = (got == ref).double().mean().item()
    print(f"C4 step_sample vs step()+sample_tokens: {same:.4f} of {ref.numel()} tokens equal, "
          f"{outside} draws outside the top-{K}", flush=True)
    assert torch.equal(got, ref)
    assert outside == 0


def test_c5_forward_logits(release):
    """C5: one fused forward at B = 8, T = 4096 (12 levels) with two document separators planted per
    row (the doc-reset mask in play) against the eager forward. fp32: rel <= 1e-4 and equal argmax;
    bf16: the model-level bf16 criterion over all 32768 positions, with the same-rounding floor."""
    cfgd, m32, m16, _, _ = release
    g = torch.Generator(device=DEV).manual_seed(6)
    ids = torch.randint(0, cfgd["vocab_size"] - 1, (8, 4096), device=DEV, generator=g)
    for r in range(8):
        ids[r, 300 + 450 * r] = cfgd["eot_token"]
        ids[r, 3500 - 97 * r] = cfgd["eot_token"]
    with torch.no_grad():
        print("C5 fp32 eager forward", flush=True)
        e32 = m32(ids).logits
        print("C5 fp32 fused forward", flush=True)
        f32 = m32.enable_fused_gates()(ids).logits
        m32.enable_fused_gates(False)
        r32 = rel_err(f32, e32)
        agree = (f32.argmax(-1) == e32.argmax(-1)).double().mean().item()
        print(f"C5 fp32 fused vs eager: rel={r32:.2e}, argmax agreement {agree:.6f}", flush=True)
        del f32
        assert r32 <= 1e-4
        assert agree == 1.0
        print("C5 bf16 eager and fused forwards", flush=True)
        e16 = m16(ids).logits.float()
        with fp32_product_accumulation():
            a16 = m16(ids).logits.float()
        f16 = m16.enable_fused_gates()(ids).logits.float()
        m16.enable_fused_gates(False)
    V = e32.shape[-1]
    bf16_vs_truth(f16.view(-1, V), e16.view(-1, V), e32.view(-1, V), "C5 bf16 B=8 T=4096", alt16=a16.view(-1, V))
