#!/usr/bin/env python3
"""Benchmark of Dispatcher-Hybrid's hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Headline (`value`): steady-state batch-1 bf16 greedy decode tok/s of the 292M model at 3840-4096
context through FusedGraphedHybridDecoder: the whole step as ONE persistent launch per token
(dh_decode_persistent_step; with --graph-step the graph of launches instead: one HIP-graph replay
per token, five gfx950 launches per tree layer -- fused RMSNorm/projections, the mixer step's gate
readouts, its recurrence fused with the out-projection + residual, RMSNorm + SwiGLU,
down-projection + residual). A step is one decode token; prefill and graph capture are outside the
timed region (reference scripts/benchmark_decode.py:21-28 protocol). Also reported in the same JSON
line:
  decode_b16_*      lockstep batch-16 decode with temperature 0.8 / top-k 50 sampling (dh_sample_topk)
  decoder_prefill_* the decoders' C3 prefill (3840 tokens, all decode state): fused vs eager
  prefill_*         C2: 292M bf16 forward at B=1, T=1024: graphed fused forward (graphed_logits), the
                    fused forward launched from the host, eager
  forward_c5_*      C5: 292M bf16 forward at B=8, T=4096: graphed fused forward (graphed_logits), the
                    fused forward launched from the host, eager (+ peak HBM of the launched ones)
  gate_path_c5_*    one mixer layer at the C5 shape, fused vs eager
  prefill_kernels_c5  the parallel path's kernels at the C5 shape, HIP-event timed, each against its
                    roofline (gate pre-activations and banded attention: MFMA; level scan: HBM)
  roofline          decode_persistent_kernel (dh_decode_persistent_step), the only kernel of a
                    batch-1 step: algorithmic bytes / HIP-event-timed launch duration (with
                    --graph-step: dh_decode_gemv's launches of the graph of launches)
  gemv_chain        dh_decode_gemv's 57 launches of the graph-of-launches step, the same measure
  mixer_step        the decoders' mixer step per tree layer at t = 4000: batch 1 dh_decode_gates +
                    dh_decode_scan_out, batch 16 dh_decode_mixer_step
  step_roofline     whole decode step: bf16 weight bytes per token x tok/s vs 8 TB/s
  parity_bf16       the north star's bf16 quantities (logit max-abs, greedy-argmax agreement) of the
                    C2 fused-gates forward and the C3 one-launch step against the eager bf16 and fp32 paths
  c1_mixer_gpu_*    C1: one fp32 mixer layer (d 512, 8 levels, T 256) through the fused path
  cpu_baseline      the oracle's eager torch path (reference algorithm) on the host CPU, fp32: C3 decode
                    (value), C2 prefill and the C1 mixer layer
All inputs are synthetic (uniform token ids) and the weights are a random init of the released
architecture. Rank 0 prints one JSON line. --leg runs one part alone (for rocprofv3 runs): see --help.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dispatcher-hybrid-2_amd"))

METRIC = "decode tok/s @4096 ctx (batch 1 & 16) + prefill tok/s; % HBM roofline"
N_PARAMS = 292_158_464                 # released config, tied head counted once
W_BYTES = 2 * N_PARAMS                 # bf16 weight bytes streamed per decode step
HBM_PEAK_GBS = 8000.0                  # MI355X HBM3E
MFMA_BF16_TFLOPS = 2500.0              # MI355X dense bf16
REF_DECODE_TOK_S = 525.1               # reference FusedGraphedHybridDecoder @3900 ctx (A6000, README.md:76-81)
REF_DECODE_BY_CTX = {256: 534.8, 1024: 534.1, 2048: 534.1, 3900: 525.1}   # same table, by context
EOT = 50256
# HBM bytes per dh_decode_gemv launch, averaged over the decode step's 57 launches: rocprofv3 --pmc
# FETCH_SIZE (x 1.99975, the factor a 256 MiB copy's reading gives) + WRITE_SIZE (x 1.0), from
# profiles/decode_c3_b1_kernels.md
TRAFFIC_GEMV_LAUNCH = 9_453_050
# HBM bytes per decode_persistent_kernel launch (one batch-1 step), same counters and factors, from
# profiles/decode_c3_b1_persistent.md
TRAFFIC_PERSISTENT_LAUNCH = 616_437_816
# algorithmic bytes of one batch-1 step at context >= 1024: weights 584,316,928 + tree state
# 1,224,704 + windowed keys and values 8,396,800
STEP_BYTES = 584_316_928 + 1_224_704 + 8_396_800


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=3840)
    ap.add_argument("--skip-extras", action="store_true", help="decode batch-1 only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph-step", action="store_true",
                    help="C3 on the graph of launches instead of the one-launch step (profiling)")
    ap.add_argument("--cpu-steps", type=int, default=32)
    ap.add_argument("--cpu-prompt", type=int, default=1024)
    ap.add_argument("--leg", default="all",
                    choices=["all", "prefill-kernels", "prefill-c2", "forward-c5", "decode-b16", "decode-trace",
                             "parity-bf16"],
                    help="prefill-kernels: only the C5 kernel timings; prefill-c2: only the C2 fused "
                         "forward (for rocprofv3 runs); forward-c5: only the C5 graphed forward (for "
                         "rocprofv3 runs); decode-b16: only the batch-16 sampling decode "
                         "(for rocprofv3 runs); decode-trace: per-phase timestamps of the one-launch "
                         "batch-1 step (wait vs work table); parity-bf16: only the bf16 parity figures")
    return ap.parse_args()


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def build_model(torch, dev):
    from dispatcher_hybrid import DispatcherConfig, DispatcherHybridForCausalLM
    torch.manual_seed(0)
    with torch.device(dev):
        model = DispatcherHybridForCausalLM(DispatcherConfig())
    return model.to(torch.bfloat16).eval()


def sync_barrier(torch):
    torch.cuda.synchronize()


def time_decode(torch, model, batch, prompt, warmup, steps, sample, persistent=True):
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(3 if batch == 1 else 4)
    ids = torch.randint(0, EOT, (1, prompt), device=dev, generator=g).expand(batch, -1).contiguous()
    dec = FusedGraphedHybridDecoder(model, persistent=persistent)
    logits = dec.prefill(ids)[:, -1]
    torch.manual_seed(5)

    if not sample:
        # greedy as fast_generate runs it: the pick (device argmax, torch.argmax's token) is the last
        # part of the captured step and feeds the next one; one graph replay per token
        dec.greedy_start(logits)
        for _ in range(warmup):
            dec.step_greedy()
        sync_barrier(torch)
        # HIP events on the stream the steps are launched on (torch's current stream): with the
        # one-launch step this is the kernel's average duration plus the small gap between launches
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            dec.step_greedy()
        e1.record()
        sync_barrier(torch)
        dt = time.perf_counter() - t0
        if dec.check_persistent():                         # a one-launch step timed out: redone, not timed
            raise RuntimeError("a one-launch decode step timed out inside the timed loop")
        dec.event_us_per_step = e0.elapsed_time(e1) * 1e3 / steps
        return batch * steps / dt, 1e3 * dt / steps, dec

    # temperature 0.8 / top-k 50 sampling on the device (draws keyed by seed, position and row) as
    # the last launch of the captured step: one graph replay per token, the sampled token feeding
    # the next replay on the device (fast_generate's sampling branch)
    dec.sample_start(logits, 0.8, 50, 5)
    for _ in range(warmup):
        dec.step_sample()
    sync_barrier(torch)
    t0 = time.perf_counter()
    for _ in range(steps):
        dec.step_sample()
    sync_barrier(torch)
    dt = time.perf_counter() - t0
    return batch * steps / dt, 1e3 * dt / steps, dec


def time_decoder_prefill(torch, model, prompt, reps=3):
    """The decoders' prefill of a C3 prompt (state for every layer plus the logits): the fused
    decoder's (parallel gate kernels fill the tree state) against the eager one the reference's
    fused decoder runs (decoding.py:143-185, 353-356). Graph capture is not included."""
    from dispatcher_hybrid.decoding import IncrementalDecoder, _FusedPrefillDecoder
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(7)
    ids = torch.randint(0, EOT, (1, prompt), device=dev, generator=g)
    res = []
    for cls in (_FusedPrefillDecoder, IncrementalDecoder):
        dec = cls(model)
        dec.prefill(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            dec.prefill(ids)
        torch.cuda.synchronize()
        res.append((time.perf_counter() - t0) / reps * 1e3)
        del dec
        torch.cuda.empty_cache()
    return res[0], res[1]


def time_forward(torch, model, ids, fused, reps=3):
    model.enable_fused_gates(fused)
    with torch.no_grad():
        model(ids)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(reps):
            model(ids)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
    peak = torch.cuda.max_memory_allocated()
    model.enable_fused_gates(False)
    return ids.numel() / dt, dt * 1e3, peak


def time_forward_graphed(torch, model, ids, reps=10):
    """The fused forward as one HIP graph replay per call (model.graphed_logits: the token ids copied
    into the graph's input buffer, then the replay), wall clock over `reps` calls after the capture."""
    model.enable_fused_gates(True)
    with torch.no_grad():
        model.graphed_logits(ids)                      # capture
        model.graphed_logits(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            model.graphed_logits(ids)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
    model.release_graphs()
    model.enable_fused_gates(False)
    return ids.numel() / dt, dt * 1e3


def time_mixer(torch, mixer, x, mask, fused, reps=5):
    """Milliseconds per mixer layer, and the layer's peak device memory above what was allocated
    before it (its activations and temporaries, bytes)."""
    mixer.use_fused_gates = fused
    with torch.no_grad():
        mixer(x, mask)
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(reps):
            mixer(x, mask)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps * 1e3
        peak = torch.cuda.max_memory_allocated() - base
    mixer.use_fused_gates = False
    return dt, peak


def _graph_time(torch, launch, n, reps):
    """Capture launch(0..n-1) back to back in one HIP graph on the current stream, replay it `reps`
    times between two HIP events recorded on that stream; average microseconds per launch. The
    figure includes the graph's inter-node gap (the per-launch floor a decode step pays)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(n, 8)):
            launch(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    del graph
    return 1e3 * e0.elapsed_time(e1) / (reps * n)


def gemv_chain_roofline(torch, model, reps=20):
    """dh_decode_gemv over the launches of one batch-1 decode step: the same 57 launches, shapes and
    weights as FusedGraphedHybridDecoder's step -- per tree layer RMSNorm + [W_in; W1x; W1s],
    RMSNorm + SwiGLU, linear_down + residual (its linear_out runs inside dh_decode_scan_out); per
    attention layer RMSNorm + [Wq; Wk; Wv], linear_out + residual, RMSNorm + SwiGLU, linear_down +
    residual; RMSNorm + lm_head -- on random activations, in one HIP graph. The model's 584 MB of
    weights exceed the 256 MB last-level cache, so every launch streams its weights from HBM as in
    decode. Returns (algorithmic bytes per step, microseconds per launch, launches)."""
    from dispatcher_hybrid import fused_step
    from dispatcher_hybrid.modeling_dispatcher import AttentionBlock
    dev = next(model.parameters()).device
    dt = torch.bfloat16
    cfg = model.config
    d, ff = cfg.d_model, cfg.dim_feedforward
    t_buf = torch.zeros(1, dtype=torch.long, device=dev)
    x = torch.randn(1, d, device=dev, dtype=dt)
    xr = torch.randn(1, d, device=dev, dtype=dt)
    h = torch.randn(1, ff, device=dev, dtype=dt) * 0.1
    o = torch.empty(1, 3 * d + ff, device=dev, dtype=dt)
    logits = torch.empty(1, model.lm_head.weight.shape[0], device=dev, dtype=dt)
    calls, nbytes = [], 0

    def add(xin, segs, **kw):
        nonlocal nbytes
        K = xin.shape[1]
        rows = sum(w.shape[0] for w, _, _, _ in segs)
        nbytes += 2 * (rows * K + K + (K if kw.get("norm_weight") is not None else 0)
                       + (rows // 2 if kw.get("swiglu") else rows) + (rows if kw.get("resid") is not None else 0))
        calls.append(lambda: fused_step.decode_gemv(xin, segs, t_buf, **kw))

    for blk in model.blocks:
        if isinstance(blk, AttentionBlock):
            at = blk.attn
            ws = [at.linear_q.weight, at.linear_k.weight, at.linear_v.weight]
            wo = at.linear_out.weight
        else:
            mx = blk.mixer
            ws = [mx.linear_in.weight, mx.gate_hidden.weight, mx.gate_hidden_src.weight]
            wo = mx.linear_out.weight
        add(x, [(w, o[:, i * d:], o.shape[1], 0) for i, w in enumerate(ws)], norm_weight=blk.norm1.weight)
        if isinstance(blk, AttentionBlock):
            add(x, [(wo, xr, d, 0)], resid=xr)
        f = blk.ffn
        add(x, [(f.linear_gate.weight, o, ff, 0), (f.linear_up.weight, o, ff, 0)],
            norm_weight=blk.norm2.weight, swiglu=True)
        add(h, [(f.linear_down.weight, xr, d, 0)], resid=xr)
    add(x, [(model.lm_head.weight, logits, logits.shape[1], 0)], norm_weight=model.norm_out.weight)
    us = _graph_time(torch, lambda i: calls[i](), len(calls), reps)
    return nbytes, us, len(calls)


def mixer_step_time(torch, model, copies=200, reps=5):
    """The decoder's mixer step per tree layer as the decoders run it, at t = 4000 (all 12 levels
    live), the weights cycling through `copies` distinct copies (more than the last-level cache):
      b1:  dh_decode_gates + dh_decode_scan_out (the batch-1 graph of launches: gate readouts, then
           the recurrence inside the out-projection + residual launch)
      b16: dh_decode_mixer_step (batch > 1: gates and recurrence in one launch per layer; the
           out-projection is a separate GEMV launch, not timed here)
    Returns {form: {us, bytes, achieved_gbs}} with algorithmic bytes per step."""
    from dispatcher_hybrid import fused_step
    dev = next(model.parameters()).device
    mx = next(b.mixer for b in model.blocks if hasattr(b, "mixer"))
    L, H, GH, d = mx.levels, mx.num_heads, mx.gate_hidden.out_features, model.config.d_model
    hd, S, Tmax, bf = d // H, (2 << mx.levels) - 2, 4096, torch.bfloat16
    Ws = [torch.stack([mx.gate_out, mx.forget_out, mx.reset_out]).clone() for _ in range(copies)]
    Wo = [mx.linear_out.weight.clone() for _ in range(copies)]
    bi, bfb, br = mx.gate_out_bias, mx.forget_out_bias, mx.reset_out_bias
    t_buf = torch.full((1,), 4000, dtype=torch.long, device=dev)
    s = 2
    out = {}
    for Bb in (1, 16):
        A = torch.randn(Bb, GH, device=dev).to(bf)
        V0 = torch.randn(Bb, d, device=dev).to(bf)
        Y = torch.empty(Bb, d, device=dev, dtype=bf)
        x = torch.randn(Bb, d, device=dev).to(bf)
        B_hist = torch.randn(Bb, Tmax, GH, device=dev).to(bf)
        rg = torch.rand(Bb, Tmax, L, H, device=dev).to(bf)
        ring = torch.randn(Bb, S, d, device=dev).to(bf)
        stage = torch.zeros(fused_step.stage_floats(Bb, H, L, hd), device=dev)
        state = Bb * (L * GH + GH + 2 * L * H + 2 * L * d + 2 * d) * s      # A, B rows, gates, ring reads/writes, V0, Y
        if Bb == 1:
            def launch(i):
                W = Ws[i % copies]
                fused_step.decode_gates_scan_out(A, B_hist, W[0], W[1], W[2], bi, bfb, br, t_buf, rg, ring, V0, Y,
                                                 stage, Wo[i % copies], x, x)
            nbytes = 3 * L * H * GH * s + 3 * L * H * s + d * d * s + state + 2 * d * s
            form = "b1", "dh_decode_gates + dh_decode_scan_out (batch 1: gates, recurrence, out-projection + residual)"
            us = 2 * _graph_time(torch, launch, copies, reps)             # two launches per step
        else:
            def launch(i):
                W = Ws[i % copies]
                fused_step.decode_mixer_step(A, B_hist, W[0], W[1], W[2], bi, bfb, br, t_buf, rg, ring, V0, Y)
            nbytes = 3 * L * H * GH * s + 3 * L * H * s + state
            form = "b16", "dh_decode_mixer_step (batch 16: gates and recurrence; out-projection not included)"
            us = _graph_time(torch, launch, copies, reps)
        out[form[0]] = {"kernels": form[1], "us": round(us, 3), "bytes": nbytes,
                        "achieved_gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
    del Ws, Wo
    torch.cuda.empty_cache()
    return out


def prefill_kernels(torch, dev, reps=10):
    """The parallel path's gfx950 kernels at the C5 shape (b 8, T 4096, GH 1024, 16 heads of 64,
    12 levels, doc mask; attention window 1024), each timed with HIP events on its launch stream over
    `reps` launches, on synthetic bf16 inputs: the activated gate pre-activations (MFMA-bound: FLOPs
    2 b T L GH 3H), the level scan (HBM: gates + V0 in, V out) and the banded attention (MFMA: 4 b H hd
    sum_t min(t+1, W) FLOPs for QK^T and PV), and the three input projections as one dh_proj_gemm
    launch (MFMA: 2 b T d (d + 2 GH) FLOPs) beside the three library GEMMs it replaces."""
    from dispatcher_hybrid import fused_attention as fa
    from dispatcher_hybrid import fused_gates as fg
    b, T, GH, H, hd, L, W = 8, 4096, 1024, 16, 64, 12, 1024
    d = H * hd
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(11)
    A = torch.randn(b, T, GH, device=dev, generator=g).to(bf)
    B = torch.randn(b, T, GH, device=dev, generator=g).to(bf)
    Ws = [(torch.randn(L, H, GH, device=dev, generator=g) / GH ** 0.5).to(bf) for _ in range(3)]
    bs = [torch.randn(L, H, device=dev, generator=g) for _ in range(3)]
    mask = (torch.rand(b, T, L, device=dev, generator=g) > 0.001).to(bf)
    V0 = torch.randn(b, T, d, device=dev, generator=g).to(bf)
    V = torch.empty_like(V0)
    buf = torch.empty((3, b, H, L, T), device=dev, dtype=bf)
    gates = [buf[i].permute(0, 3, 2, 1) for i in range(3)]
    q, k, v = (torch.randn(b, T, d, device=dev, generator=g).to(bf) for _ in range(3))
    ang = torch.outer(torch.arange(T, device=dev, dtype=torch.float32),
                      torch.pow(10000.0, -torch.arange(0, hd, 2, device=dev, dtype=torch.float32) / hd))
    cos, sin = ang.cos().to(bf), ang.sin().to(bf)

    def timed(fn):
        for _ in range(2):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    xin = torch.randn(b, T, d, device=dev, generator=g).to(bf)
    Wp = [(torch.randn(n, d, device=dev, generator=g) / d ** 0.5).to(bf) for n in (d, GH, GH)]
    proj_us = timed(lambda: fg.fused_projections(xin, Wp))
    lib_us = timed(lambda: [torch.nn.functional.linear(xin, w) for w in Wp])
    gate_us = timed(lambda: fg._preacts_launch(A, B, *Ws, *bs, mask, gates, gates[0].stride(), 1, L, "bench"))
    scan_us = timed(lambda: fg._scan_launch(*gates, None, V0, V, H, L, True, "bench"))
    attn_us = timed(lambda: fa.window_attention(q, k, v, cos, sin, H, W))
    gate_fl = 2 * b * T * L * GH * 3 * H
    gate_bytes = 2 * (2 * b * T * GH + 3 * L * H * GH + 3 * b * T * L * H + b * T * L)
    scan_bytes = 2 * (3 * b * T * L * H + 2 * b * T * d)
    attn_fl = 4 * b * H * hd * sum(min(t + 1, W) for t in range(T))
    tf = lambda fl, us: fl / (us * 1e-6) / 1e12
    gb = lambda by, us: by / (us * 1e-6) / 1e9
    proj_fl = 2 * b * T * d * (d + 2 * GH)
    return {
        "shape": f"b {b}, T {T}, GH {GH}, {H} heads x {hd}, {L} levels, window {W}, bf16",
        "input_projections": {"us": round(proj_us, 1), "bound": "mfma", "achieved": round(tf(proj_fl, proj_us), 1),
                              "peak": MFMA_BF16_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(tf(proj_fl, proj_us) / MFMA_BF16_TFLOPS, 4), "flops": proj_fl,
                              "three_library_gemms_us": round(lib_us, 1),
                              "product_runs": "the three library GEMMs (above PROJ_GEMM_MAX_ROWS = 8192 rows; "
                                              "dh_proj_gemm at or below)"},
        "gate_preacts": {"us": round(gate_us, 1), "bound": "mfma", "achieved": round(tf(gate_fl, gate_us), 1),
                         "peak": MFMA_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf(gate_fl, gate_us) / MFMA_BF16_TFLOPS, 4),
                         "hbm_gbs": round(gb(gate_bytes, gate_us), 1), "flops": gate_fl, "bytes": gate_bytes},
        "level_scan": {"us": round(scan_us, 1), "bound": "hbm", "achieved": round(gb(scan_bytes, scan_us), 1),
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gb(scan_bytes, scan_us) / HBM_PEAK_GBS, 4),
                       "bytes": scan_bytes},
        "window_attention": {"us": round(attn_us, 1), "bound": "mfma", "achieved": round(tf(attn_fl, attn_us), 1),
                             "peak": MFMA_BF16_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tf(attn_fl, attn_us) / MFMA_BF16_TFLOPS, 4), "flops": attn_fl},
    }


def copy_probe(torch, dev, mib=256):
    """One plain device-to-device copy of `mib` MiB (read once, written once). Under rocprofv3
    --pmc its FETCH_SIZE / WRITE_SIZE readings turn those counters into bytes for the other
    kernels of the same run."""
    a = torch.zeros(mib << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def decode_trace(torch, model, prompt, warmup, steps):
    """Per-phase timing of the one-launch batch-1 step (dh_decode_persistent_trace) over `steps`
    greedy steps after `warmup` untraced ones. Per phase of a step: the critical-path increment (the
    latest workgroup's end minus the previous phase's), the median workgroup's wait (start to the
    end of its wait for other workgroups' words) and work (wait end to phase end), and the spread
    of the wait ends over workgroups; averaged by phase kind over layers and steps (microseconds)."""
    import numpy as np

    from dispatcher_hybrid import fused_step
    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder
    dev = next(model.parameters()).device
    ids = torch.randint(0, EOT, (1, prompt), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    dec = FusedGraphedHybridDecoder(model)
    dec.greedy_start(dec.prefill(ids)[:, -1])
    for _ in range(warmup):
        dec.step_greedy()
    if not dec._pers:
        raise SystemExit("decode-trace: the one-launch step is not used for this model")
    kinds = dec._pers["kinds"]
    nph = fused_step.persistent_phases(kinds)
    grid = torch.cuda.get_device_properties(dev).multi_processor_count
    tr = torch.zeros(steps, grid, nph, 3, dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    for i in range(steps):
        dec._persistent_step(trace=tr[i])
        dec.t += 1
    torch.cuda.synchronize()
    if dec.check_persistent():
        raise SystemExit("decode-trace: a traced step timed out")
    a = tr.cpu().numpy().astype(np.float64) / 100.0                 # 100 MHz counter -> us
    names = []
    for k in kinds:
        names += ["in-projection", "gate readouts", "recurrence + out-projection"] if k == 0 else \
                 ["attention q/k/v", "attention segments", "attention combine", "attention out-projection"]
        names += ["feed-forward up", "feed-forward down"]
    names += ["vocabulary head", "greedy pick"]
    start, ready, end = a[..., 0], a[..., 1], a[..., 2]
    end_max = end.max(axis=1)                                       # (steps, nph)
    t0 = np.where(start[:, :, 0] > 0, start[:, :, 0], np.inf).min(axis=1)
    inc = np.diff(np.concatenate([t0[:, None], end_max], axis=1), axis=1)
    rows = {}
    for p_, nm in enumerate(names):
        live = ready[:, :, p_] > 0
        w = np.where(live, ready[:, :, p_] - start[:, :, p_], np.nan)
        k_ = np.where(live, end[:, :, p_] - ready[:, :, p_], np.nan)
        sp = np.where(live, ready[:, :, p_], np.nan)
        spread = np.nanmax(sp, axis=1) - np.nanmin(sp, axis=1)
        r = rows.setdefault(nm, {"n": 0, "span": 0.0, "wait": 0.0, "work": 0.0, "spread": 0.0})
        r["n"] += 1
        r["span"] += float(inc[:, p_].mean())
        r["wait"] += float(np.nanmean(np.nanmedian(w, axis=1)))
        r["work"] += float(np.nanmean(np.nanmedian(k_, axis=1)))
        r["spread"] += float(np.nanmean(spread))
    table = []
    for nm, r in rows.items():
        table.append({"phase": nm, "per_step": r["n"], "span_us": round(r["span"] / r["n"], 3),
                      "wait_us": round(r["wait"] / r["n"], 3), "work_us": round(r["work"] / r["n"], 3),
                      "ready_spread_us": round(r["spread"] / r["n"], 3),
                      "span_total_us": round(r["span"], 2)})
    total = float((end_max[:, -1] - t0).mean())
    return {"step_us": round(total, 2), "phases": nph, "workgroups": grid, "steps": steps,
            "context": f"{prompt + warmup}-{prompt + warmup + steps}", "table": table}


def _cpu_threads():
    """Threads for the CPU legs: the process's affinity set, capped at the OMP_NUM_THREADS share the
    host grants one GPU's job (16 on the GPU boxes here)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else n


def _cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(torch, model, prompt, steps):
    """The oracle's eager torch path (the reference's eager algorithm) in fp32 on the host cores:
    C3 decode (the reported baseline), plus the C1 mixer layer and the C2 prefill rows."""
    sys.path.insert(0, ROOT)
    from oracle import torch_eager
    n = _cpu_threads()
    torch.set_num_threads(n)
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    if "lm_head.weight" not in sd:
        sd["lm_head.weight"] = sd["embedding.weight"]
    spec = torch_eager.Spec(model.config)
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, EOT, (1, prompt), generator=g)
    dec = torch_eager.EagerDecoder(sd, spec)
    logits = dec.prefill(ids)[:, -1]
    logits = dec.step(logits.argmax(-1))                    # warm-up step
    t0 = time.perf_counter()
    for _ in range(steps):
        logits = dec.step(logits.argmax(-1))
    dt = time.perf_counter() - t0
    del dec
    # C2: the 292M forward over 1024 tokens (one warm-up, one timed run)
    ids2 = torch.randint(0, 50257, (1, 1024), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        torch_eager.forward(sd, spec, ids2)
        t0 = time.perf_counter()
        torch_eager.forward(sd, spec, ids2)
        c2 = time.perf_counter() - t0
    del sd
    c1 = c1_cpu(torch, torch_eager)
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": n, "kind": "port",
            "sample": f"fp32 eager decode (oracle/torch_eager.EagerDecoder, reference algorithm), "
                      f"batch 1, {steps} timed steps after a {prompt}-token prefill (per-token cost "
                      f"is flat in context past the tree's O(log t) reads); {n} threads of host CPU: "
                      f"{_cpu_model_name()}",
            "c2_prefill_tok_s": round(1024 / c2, 1),
            "c2_sample": "fp32 eager forward of the 292M model over 1024 tokens (oracle/torch_eager.forward), "
                         "one timed run after a warm-up",
            "c1_mixer_ms": round(c1, 3),
            "c1_sample": "one mixer layer, d 512, 8 heads, 8 levels, T 256, fp32, x ~ N(0,1), weights "
                         "N(0, 0.02), biases 0 (oracle/torch_eager.mixer): median of 7 runs"}


def _c1_layer(torch):
    """The C1 single mixer layer (d 512, 8 heads of 64, 8 levels, T 256): state dict, input, mask."""
    g = torch.Generator().manual_seed(1)
    d, H, L, T = 512, 8, 8, 256
    w = lambda *shape: torch.randn(*shape, generator=g) * 0.02
    sd = {"m.linear_in.weight": w(d, d), "m.gate_hidden.weight": w(d, d), "m.gate_hidden_src.weight": w(d, d),
          "m.linear_out.weight": w(d, d), "m.gate_out": w(L, H, d), "m.forget_out": w(L, H, d),
          "m.reset_out": w(L, H, d), "m.gate_out_bias": torch.zeros(L, H),
          "m.forget_out_bias": torch.zeros(L, H), "m.reset_out_bias": torch.zeros(L, H)}
    x = torch.randn(1, T, d, generator=torch.Generator().manual_seed(0))
    t = torch.arange(T).unsqueeze(1)
    lag = torch.tensor([1 << l for l in range(L)])
    mask = ((t >= lag) & (lag < T)).float()
    return sd, x, mask


def c1_cpu(torch, torch_eager):
    from dispatcher_hybrid import DispatcherConfig
    sd, x, mask = _c1_layer(torch)
    spec = torch_eager.Spec(DispatcherConfig(d_model=512, num_heads=8, max_len=256, num_layers=1, attn_layers=(),
                                             vocab_size=512, dim_feedforward=1024))
    with torch.no_grad():
        torch_eager.mixer(sd, "m.", x, mask, spec)
        ts = []
        for _ in range(7):
            t0 = time.perf_counter()
            torch_eager.mixer(sd, "m.", x, mask, spec)
            ts.append(time.perf_counter() - t0)
    return sorted(ts)[3] * 1e3


def c1_gpu(torch, dev, reps=20):
    """The C1 layer (fp32) through the fused mixer on the GPU: milliseconds per layer."""
    from dispatcher_hybrid import DispatcherConfig
    from dispatcher_hybrid.modeling_dispatcher import DispatcherMixer
    sd, x, mask = _c1_layer(torch)
    mx = DispatcherMixer(DispatcherConfig(d_model=512, num_heads=8, max_len=256, num_layers=1, attn_layers=(),
                                          vocab_size=512, dim_feedforward=1024))
    mx.load_state_dict({k[2:]: v for k, v in sd.items()})
    mx = mx.to(dev).eval()
    mx.use_fused_gates = True
    x, mask = x.to(dev), mask.to(dev)
    with torch.no_grad():
        for _ in range(3):
            mx(x, mask)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            mx(x, mask)
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps * 1e3


def _agreement(torch, fused16, eager16, truth32):
    """The north-star bf16 quantities of fused bf16 logits (n, V): max-abs and raw greedy-argmax
    agreement against the eager bf16 path, the same against the fp32 eager path for both bf16 paths,
    and argmax agreement where the fp32 path's top-2 margin exceeds 0.1 (decisive positions)."""
    top2 = torch.topk(truth32, 2, dim=-1).values
    decisive = (top2[..., 0] - top2[..., 1]) > 0.1
    agree32 = fused16.argmax(-1) == truth32.argmax(-1)
    return {"max_abs_vs_eager_bf16": round((fused16 - eager16).abs().max().item(), 4),
            "argmax_vs_eager_bf16": round((fused16.argmax(-1) == eager16.argmax(-1)).double().mean().item(), 4),
            "max_abs_vs_eager_fp32": round((fused16 - truth32).abs().max().item(), 4),
            "eager_bf16_max_abs_vs_eager_fp32": round((eager16 - truth32).abs().max().item(), 4),
            "argmax_vs_eager_fp32": round(agree32.double().mean().item(), 4),
            "argmax_vs_eager_fp32_decisive": round(agree32[decisive].double().mean().item(), 4)
            if bool(decisive.any()) else None,
            "decisive_positions": int(decisive.sum()), "positions": int(decisive.numel())}


def _floor(torch, alt16, eager16, fused16):
    """max-abs and raw greedy-argmax agreement of two eager bf16 runs at the same rounding points, and
    the fused path's max-abs against the eager bf16 path as a multiple of that floor (the tests
    require <= 2)."""
    mx = (alt16 - eager16).abs().max().item()
    return {"max_abs": round(mx, 4), "mean_abs": round((alt16 - eager16).abs().mean().item(), 5),
            "argmax_agree": round((alt16.argmax(-1) == eager16.argmax(-1)).double().mean().item(), 4),
            "fused_max_abs_over_floor": round((fused16 - eager16).abs().max().item() / mx, 3)}


def parity_bf16(torch, model, prompt, steps=256):
    """bf16 parity figures of the measured paths on the bench's own inputs: C2 (fused-gates forward,
    T = 1024) and C3 (the one-launch greedy step over `steps` positions from the bench's context,
    teacher-forcing the eager decoders with its tokens).

    same_rounding_floor: the eager bf16 path against itself with only the accumulation order of its
    matrix products changed (dispatcher_hybrid.numerics.fp32_product_accumulation: each bf16 product
    as an fp32 product of the same bf16 operands, rounded once) -- the logit max-abs and argmax
    agreement that any bf16 implementation with its own GEMM kernels can be expected to reach
    against the eager bf16 path."""
    import copy

    from dispatcher_hybrid.decoding import FusedGraphedHybridDecoder, IncrementalDecoder
    from dispatcher_hybrid.numerics import fp32_product_accumulation
    dev = next(model.parameters()).device
    m32 = copy.deepcopy(model).float()
    g = torch.Generator(device=dev).manual_seed(2)
    ids = torch.randint(0, 50257, (1, 1024), device=dev, generator=g)
    with torch.no_grad():
        e16 = model(ids).logits[0].float()
        with fp32_product_accumulation():
            a16 = model(ids).logits[0].float()
        f16 = model.enable_fused_gates()(ids).logits[0].float()
        model.enable_fused_gates(False)
        e32 = m32(ids).logits[0].float()
    out = {"c2": _agreement(torch, f16, e16, e32)}
    out["c2"]["same_rounding_floor"] = _floor(torch, a16, e16, f16)
    del e16, f16, e32, a16
    steps = min(steps, model.config.max_len - prompt)
    ids = torch.randint(0, EOT, (1, prompt), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    dec = FusedGraphedHybridDecoder(model)
    dec.greedy_start(dec.prefill(ids)[:, -1])
    got = []
    for _ in range(steps):
        dec.step_greedy()
        got.append(dec.logits_out[0].float().clone())
    toks = dec.tok_hist[:, prompt:prompt + steps]
    used = bool(dec._pers)
    del dec

    def forced(m):
        d_ = IncrementalDecoder(m)
        d_.prefill(ids)
        return torch.stack([d_.step(toks[:, j])[0].float() for j in range(steps)])

    e16 = forced(model)
    with fp32_product_accumulation():
        a16 = forced(model)
    got = torch.stack(got)
    out["c3"] = _agreement(torch, got, e16, forced(m32))
    out["c3"]["same_rounding_floor"] = _floor(torch, a16, e16, got)
    out["c3"]["path"] = "one-launch step" if used else "graph of launches"
    out["c3"]["context"] = f"{prompt}..{prompt + steps - 1}"
    del m32
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.leg == "prefill-kernels":
        copy_probe(torch, dev)                  # scale reference for counter runs
        pk = prefill_kernels(torch, dev)
        log("C5 prefill kernels: " + ", ".join(f"{k} {v['us']} us" for k, v in pk.items() if isinstance(v, dict)))
        print(json.dumps({"prefill_kernels_c5": pk}), flush=True)
        return
    copy_probe(torch, dev)
    model = build_model(torch, dev)
    max_len = model.config.max_len
    if args.leg == "decode-trace":
        res = decode_trace(torch, model, min(args.prompt, max_len - args.warmup - args.steps), args.warmup, args.steps)
        for r in res["table"]:
            log(f"{r['phase']:28s} x{r['per_step']:2d}  span {r['span_us']:6.2f}  wait {r['wait_us']:6.2f}  "
                f"work {r['work_us']:6.2f}  spread {r['ready_spread_us']:6.2f}  total {r['span_total_us']:7.1f}")
        log(f"step {res['step_us']} us over {res['phases']} phases")
        print(json.dumps({"decode_trace": res}), flush=True)
        return
    if args.leg == "prefill-c2":
        g = torch.Generator(device=dev).manual_seed(2)
        ids = torch.randint(0, 50257, (1, 1024), device=dev, generator=g)
        g_tok, g_ms = time_forward_graphed(torch, model, ids)
        f_tok, f_ms, _ = time_forward(torch, model, ids, True, reps=5)
        log(f"C2 prefill: graphed {g_tok:.0f} tok/s ({g_ms:.3f} ms), fused forward launched from the host "
            f"{f_tok:.0f} tok/s ({f_ms:.3f} ms)")
        print(json.dumps({"prefill_tok_s": round(g_tok, 1), "prefill_ms": round(g_ms, 3),
                          "prefill_host_launched_tok_s": round(f_tok, 1), "prefill_host_launched_ms": round(f_ms, 3)}),
              flush=True)
        return
    if args.leg == "forward-c5":
        g = torch.Generator(device=dev).manual_seed(6)
        ids = torch.randint(0, 50257, (8, 4096), device=dev, generator=g)
        ids[:, 1000] = EOT
        gc_tok, gc_ms = time_forward_graphed(torch, model, ids, reps=3)
        log(f"C5 forward: graphed {gc_tok:.0f} tok/s ({gc_ms:.2f} ms)")
        print(json.dumps({"forward_c5_tok_s": round(gc_tok, 1), "forward_c5_ms": round(gc_ms, 3)}), flush=True)
        return
    if args.leg == "parity-bf16":
        res = parity_bf16(torch, model, min(args.prompt, max_len - 256))
        log(f"bf16 parity: {json.dumps(res)}")
        print(json.dumps({"parity_bf16": res}), flush=True)
        return
    if args.leg == "decode-b16":
        steps16 = min(args.steps, 128)
        p16 = min(args.prompt, max_len - args.warmup - steps16)
        tok16, ms16, _ = time_decode(torch, model, 16, p16, args.warmup, steps16, sample=True)
        log(f"C4 decode B=16: {tok16:.1f} tok/s ({ms16:.3f} ms/step)")
        print(json.dumps({"decode_b16_tok_s": round(tok16, 1), "decode_b16_ms_per_step": round(ms16, 4)}), flush=True)
        return
    prompt = min(args.prompt, max_len - args.warmup - args.steps)
    if prompt < 1:
        raise SystemExit("--steps + --warmup exceed the 4096-token context")
    log(f"C3 decode: B=1 prompt={prompt} warmup={args.warmup} steps={args.steps}")
    tok_s, ms_step, dec1 = time_decode(torch, model, 1, prompt, args.warmup, args.steps, sample=False,
                                       persistent=not args.graph_step)
    log(f"C3 decode: {tok_s:.1f} tok/s ({ms_step * 1e3:.1f} us/token)")
    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(tok_s / REF_DECODE_TOK_S, 3), "dtype": "bf16",
        "data": "synthetic: uniform random token ids; random init of the released 292M architecture",
        "config": {"workload": "C3: 292M bf16 batch-1 greedy decode via FusedGraphedHybridDecoder, "
                               f"prompt {prompt} then {args.warmup}+{args.steps} steps "
                               f"(context {prompt}-{prompt + args.warmup + args.steps})",
                   "batch": 1, "prompt_len": prompt, "max_len": max_len,
                   "step": "one launch per token (dh_decode_persistent_step)" if dec1._pers
                           else "graph of launches (dh_decode_gemv, dh_decode_gates, ...)"},
        "vs_baseline_ref": "reference FusedGraphedHybridDecoder 525.1 tok/s @3900 ctx on A6000 (README.md:76-81)",
    }
    step_gbs = W_BYTES * tok_s / 1e9
    out["step_roofline"] = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                            "what": "bf16 weight bytes per decode token (584,316,928 B) x tok/s"}

    out["mixer_step"] = mixer_step_time(torch, model)
    log("mixer step per tree layer: " + ", ".join(f"{k} {v['us']} us" for k, v in out["mixer_step"].items()))
    if dec1._pers:
        # the dominant (only) kernel of the step: algorithmic bytes = every weight once, the tree
        # state rows and the windowed keys and values of one token (full-byte definition)
        us = dec1.event_us_per_step
        ach = STEP_BYTES / (us * 1e-6) / 1e9
        out["roofline"] = {"kernel": "decode_persistent_kernel: one batch-1 decode step per launch "
                                     "(dh_decode_persistent_step)",
                           "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_PERSISTENT_LAUNCH,
                           "bytes_per_launch": STEP_BYTES, "avg_launch_us": round(us, 3)}
        log(f"one-launch step: {us:.1f} us/launch, {ach:.0f} GB/s")
    nbytes, avg_us, nl = gemv_chain_roofline(torch, model)
    achieved = nbytes / nl / (avg_us * 1e-6) / 1e9
    out["gemv_chain" if dec1._pers else "roofline"] = {
        "kernel": "dh_decode_gemv: the 57 launches of one batch-1 decode step (decode_gemv_row_kernel "
                  "instantiations; the graph-of-launches step)",
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_GEMV_LAUNCH,
        "bytes_per_launch": round(nbytes / nl), "bytes_per_step": nbytes,
        "avg_launch_us": round(avg_us, 3), "launches_per_step": nl}
    log(f"decode GEMV chain: {nl} launches, {avg_us:.2f} us/launch, {achieved:.0f} GB/s")
    del dec1
    torch.cuda.empty_cache()

    if not args.skip_extras:
        steps16 = min(args.steps, 128)
        p16 = min(args.prompt, max_len - args.warmup - steps16)
        tok16, ms16, d16 = time_decode(torch, model, 16, p16, args.warmup, steps16, sample=True)
        del d16
        log(f"C4 decode B=16: {tok16:.1f} tok/s")
        out["decode_b16_tok_s"] = round(tok16, 1)
        out["decode_b16_ms_per_step"] = round(ms16, 4)
        out["decode_b16_step_roofline_frac"] = round(W_BYTES * tok16 / 16 / 1e9 / HBM_PEAK_GBS, 4)

        pf_ms, pe_ms = time_decoder_prefill(torch, model, prompt)
        out["decoder_prefill_c3_fused_ms"] = round(pf_ms, 3)
        out["decoder_prefill_c3_eager_ms"] = round(pe_ms, 3)
        out["decoder_prefill_c3_speedup"] = round(pe_ms / pf_ms, 2)
        log(f"C3 decoder prefill ({prompt} tokens): fused {pf_ms:.1f} ms, eager {pe_ms:.1f} ms")

        g = torch.Generator(device=dev).manual_seed(2)
        ids = torch.randint(0, 50257, (1, 1024), device=dev, generator=g)
        # the product's prefill: the fused forward as one HIP graph replay (model.graphed_logits);
        # the same forward launched op by op from the host, and the eager (unfused) forward, beside it
        g_tok, g_ms = time_forward_graphed(torch, model, ids)
        f_tok, f_ms, _ = time_forward(torch, model, ids, True, reps=5)
        e_tok, e_ms, _ = time_forward(torch, model, ids, False, reps=5)
        flops = 2 * N_PARAMS * 1024          # weight matmuls; the mixer gate readout adds ~2%
        out["prefill_tok_s"] = round(g_tok, 1)
        out["prefill_host_launched_tok_s"] = round(f_tok, 1)
        out["prefill_eager_tok_s"] = round(e_tok, 1)
        out["prefill_speedup_vs_eager"] = round(g_tok / e_tok, 3)
        out["prefill_mfma_frac"] = round(flops / (g_ms * 1e-3) / 1e12 / MFMA_BF16_TFLOPS, 4)
        log(f"C2 prefill: graphed {g_tok:.0f} tok/s, fused launched from the host {f_tok:.0f} tok/s, "
            f"eager {e_tok:.0f} tok/s")

        # batch-1 greedy decode at the reference README's contexts (flat in context: the tree reads
        # O(log t) state and attention a fixed window); 3900 runs the 196 steps that fit max_len
        ctx = {}
        for p_ctx, ref in REF_DECODE_BY_CTX.items():
            n_ctx = min(128, 4096 - p_ctx - 16) if p_ctx != 3900 else 196 - 16
            tk, _, _ = time_decode(torch, model, 1, p_ctx, 16, n_ctx, sample=False)
            ctx[str(p_ctx)] = {"tok_s": round(tk, 1), "steps": n_ctx, "vs_reference": round(tk / ref, 3)}
        out["decode_b1_by_context"] = ctx
        log("C3 decode by context: " + ", ".join(f"{k}: {v['tok_s']} tok/s" for k, v in ctx.items()))

        g = torch.Generator(device=dev).manual_seed(6)
        ids = torch.randint(0, 50257, (8, 4096), device=dev, generator=g)
        ids[:, 1000] = EOT
        f_tok, f_ms, f_peak = time_forward(torch, model, ids, True, reps=2)
        e_tok, e_ms, e_peak = time_forward(torch, model, ids, False, reps=2)
        gc_tok, _ = time_forward_graphed(torch, model, ids, reps=3)
        out["forward_c5_tok_s"] = round(gc_tok, 1)
        out["forward_c5_host_launched_tok_s"] = round(f_tok, 1)
        out["forward_c5_eager_tok_s"] = round(e_tok, 1)
        out["forward_c5_speedup_vs_eager"] = round(gc_tok / e_tok, 3)
        out["forward_c5_peak_gb"] = round(f_peak / 1e9, 2)
        out["forward_c5_eager_peak_gb"] = round(e_peak / 1e9, 2)
        log(f"C5 forward: graphed {gc_tok:.0f} tok/s, fused launched from the host {f_tok:.0f} tok/s "
            f"({f_peak / 1e9:.1f} GB), eager {e_tok:.0f} tok/s ({e_peak / 1e9:.1f} GB)")

        mixer = next(b.mixer for b in model.blocks if hasattr(b, "mixer"))
        x = torch.randn(8, 4096, 1024, device=dev, dtype=torch.bfloat16, generator=g)
        mask = model._tree_mask(ids, 4096)
        fm, fpk = time_mixer(torch, mixer, x, mask, True)
        em, epk = time_mixer(torch, mixer, x, mask, False)
        out["gate_path_c5_fused_ms"] = round(fm, 3)
        out["gate_path_c5_eager_ms"] = round(em, 3)
        out["gate_path_c5_speedup"] = round(em / fm, 2)
        out["gate_path_c5_fused_peak_gb"] = round(fpk / 1e9, 3)
        out["gate_path_c5_eager_peak_gb"] = round(epk / 1e9, 3)
        log(f"C5 mixer layer: fused {fm:.2f} ms ({fpk / 1e9:.2f} GB), eager {em:.2f} ms ({epk / 1e9:.2f} GB)")
        del x, mask, ids
        torch.cuda.empty_cache()
        pk = prefill_kernels(torch, dev)
        out["prefill_kernels_c5"] = pk
        log("C5 prefill kernels: " + ", ".join(f"{k} {v['us']} us" for k, v in pk.items() if isinstance(v, dict)))
        out["c1_mixer_gpu_fp32_ms"] = round(c1_gpu(torch, dev), 4)
        out["parity_bf16"] = parity_bf16(torch, model, min(args.prompt, max_len - 256))
        log(f"bf16 parity: {json.dumps(out['parity_bf16'])}")

    if not args.no_cpu_baseline:
        log("CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(torch, model, args.cpu_prompt, args.cpu_steps)
        cb = out["cpu_baseline"]
        log(f"CPU baseline: C3 {cb['value']} tok/s, C2 {cb['c2_prefill_tok_s']} tok/s, C1 {cb['c1_mixer_ms']} ms "
            f"on {cb['cores']} threads")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
