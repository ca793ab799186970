#!/usr/bin/env python
"""Benchmark of the gated delta-rule core on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle S] [--no-cpu-baseline]

Headline (the JSON line's `value`): chunked GDN prefill of the 340M layer
shape, B=8 T=4096 H=8 dk=dv=128, chunk 64, bf16 q/k/v, fp32 gates / beta /
states (entry state 0.1 N(0,1)); a step is one `chunk_gated_delta_rule` call
over the whole batch with its inputs resident in HBM; value = tokens/s
(B*T tokens per step).  Three copies of the inputs (3 x 218 MB) are rotated
so that no step finds its operands in the 256 MB Infinity Cache.  Before
the timed headline steps, a fixed clock-settle phase (--settle, default 2 s of
untimed steps on the same rotating copies, right before the warmup, reported
as settle_s) brings the GPU's clocks to their loaded state, so a short
--warmup times the same level as a long one; each later event-timed leg first
runs its own operation untimed for LEG_SETTLE_S (0.3 s, reported as
leg_settle_s).

The prefill runs as two kernels per call: chunk_prep (every (chunk, head) in
parallel: the intra-chunk Q K^T and K K^T products and the triangular
inverse) and chunk_state (chunk_pipe_kernel: the sequential chunk recurrence
per (sequence, head, dv tile), with the outputs computed one chunk behind by
waves of their own), the dominant one.  The timed steps issue them as
vgdr_chunk_prep + vgdr_chunk_state with an event in between (identical GPU
work to vgdr_chunk_fwd), so each kernel has its own event-timed duration.

Also reported on the same line:
  roofline      chunk_state's achieved algorithmic TFLOP/s over bf16 dense MFMA
                peak: 6 dk dv + 4 C dv FLOP per token-head (the three state
                products and the two intra-chunk products with V) per launch,
                over its event-timed average duration; `traffic` = its measured
                HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE scaled
                by a plain-copy calibration, profiles/traffic.json) when one was
                measured on the current kernel sources, else null
  path          both kernels together against the reference's own count,
                forward chunk_scan_flops / 3 = 180,224 FLOP per token-head
  decode        one recurrent decode step at the 1.3B layer shape (B=64 H=16
                dk=dv=128) for each of 24 layer states (1.5 GB), the 24 launches
                replayed from a HIP graph; per-layer time in algorithmic GB/s
                (132,104 B per sequence-head) over 8 TB/s
  layer_kernels the layer's other kernels: the short conv + SiLU over one
                projection and the RMSNorm x SiLU(gate) output epilogue at the
                340M prefill shape (GB/s over HBM peak), and the fully fused
                decode step (conv + caches, L2 norm, beta sigmoid, recurrence,
                epilogue) at the decode shape
  backward      the chunked backward at the headline shape (all six
                gradients), against the reference's count for the backward:
                2 x 180,224 FLOP per token-head (chunk_scan_flops counts
                forward + backward as 3 x the forward); and the training pair
                (saving forward + saved backward) against 3 x 180,224; the
                same for KDA (per-channel gate) at the KDA prefill shape, with
                the token-walk backward timed beside it
  generation    the 1.3B-shape GDN LM (24 layers, d2048, vocab 32000, bf16):
                ragged prefill of 64 prompts U[64, 2048], then 256 greedy
                decode steps replayed from a HIP graph: prefill tok/s,
                generated tok/s, per-step time and the step's bytes (states
                132,104 B per sequence-head-layer, plus the weights) per second
  kda, varlen   KDA prefill (B=4 T=8192 H=8) and packed GDN prefill (32
                segments U[128, 8192], H=16) tokens/s and TFLOP/s
  cpu_baseline  the oracle's torch fp32 chunk form (the reference's CPU path)
                over the full headline workload on the host cores
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0          # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0              # MI355X HBM3E
DK = DV = 128
CHUNK = 64
FLOP_PER_TOKEN_HEAD = 180224       # chunk_scan_flops(128, 128, 64, True) / 3 (the reference's count)
PREFILL_BYTES_PER_TOKEN_HEAD = 1032
DECODE_BYTES_PER_SEQ_HEAD = 132104
# chunk_state per token-head: (K*G) S, (Q*G) S, (K*Gend)^T U~ (2 dk dv each) + TE X, A U~ (2 C dv each)
STATE_FLOP_PER_TOKEN_HEAD = 6 * DK * DV + 4 * CHUNK * DV                    # 131,072
# chunk_state bytes per token-head: q, k, v (bf16), scalar g, TE + A blocks (2 C^2 bf16 per chunk),
# o (bf16), entry + final state (2 dk dv fp32 per sequence-head, amortised over T = 4096)
STATE_BYTES_PER_TOKEN_HEAD = 2 * (2 * DK + DV) + 4 + 2 * 2 * CHUNK + 2 * DV + 2 * DK * DV * 4 // 4096
# graph-replayed legs (decode, layer kernels): timed replays (at least; --steps when larger) and
# untimed replays before them, each replay 24 launches
GRAPH_REPLAYS = 30
GRAPH_WARM_REPLAYS = 10
# default clock-settle phase: back-to-back headline prefill steps right before the warmup, outside
# the timed region (short runs after an idle GPU otherwise time the first steps up to 8% slow)
SETTLE_S = 2.0
# each later timed leg first runs its own operation, untimed, for this long (a leg
# that follows a different workload otherwise timed its first calls up to 8 % slow)
LEG_SETTLE_S = 0.3


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def bench_prefill(torch, ops, workloads, name, steps, warmup, copies=3, settle_s=0.0):
    """Timed chunked prefill.  `settle_s` seconds of untimed steps on the same
    rotating copies come first (clock settle, right before the warmup: an idle
    GPU, such as while the copies are generated, drops its clocks), then
    `warmup` untimed steps.  Each step issues chunk_prep, an event, then
    chunk_state and another event on the current stream; returns host-clock
    totals and the two kernels' event-timed durations.  Two events per step,
    around the state kernel: a third at each step's start cost about 3 us per
    step (161.1 against 158.3 us at gdn_340m; 151.1 with no events), so the
    prep time is the interval from the previous step's end to the state
    kernel's start (chunk_prep plus the launch gap before it), over steps
    1 .. K - 1."""
    xs = [workloads.workload(name, device='cuda') for _ in range(copies)]
    x0 = xs[0]
    gate = 'none' if x0.g is None else ('vector' if x0.g.dim() == 4 else 'scalar')

    def step(i, mid=None):
        x = xs[i % copies]
        ops.chunk_scan(x.q, x.k, x.v, x.g, x.beta, gate=gate, delta=True, initial_state=x.initial_state,
                       output_final_state=True, cu_seqlens=x.cu_seqlens, phase_event=mid)

    settled = 0.0
    if settle_s > 0:
        t0 = time.perf_counter()
        i = 0
        while time.perf_counter() - t0 < settle_s:
            for _ in range(20):
                step(i)
                i += 1
            torch.cuda.synchronize()
        settled = time.perf_counter() - t0
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        m, b = ev[i]
        step(i, m)
        b.record(stream)
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    prep_ms = [ev[i - 1][1].elapsed_time(ev[i][0]) for i in range(1, steps)] or [0.0]
    state_ms = [m.elapsed_time(b) for m, b in ev]
    tokens = x0.q.shape[0] * x0.q.shape[1]
    H = x0.q.shape[2]
    del xs
    op_ms = statistics.mean(p + q for p, q in zip(prep_ms, state_ms))
    return dict(tokens=tokens, H=H, total_s=total, tok_s=steps * tokens / total, settle_s=settled,
                prep_ms=statistics.mean(prep_ms), state_ms=statistics.mean(state_ms), op_ms=op_ms,
                path_tflops=tokens * H * FLOP_PER_TOKEN_HEAD / (op_ms * 1e-3) / 1e12,
                state_tflops=tokens * H * STATE_FLOP_PER_TOKEN_HEAD / (statistics.mean(state_ms) * 1e-3) / 1e12)


def time_steps(torch, fn, steps, warmup, rotate):
    """`warmup` untimed steps, then exactly `steps` timed ones; returns (host
    seconds around synchronize, per-step event ms)."""
    for i in range(warmup):
        fn(i % rotate)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        fn(i % rotate)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, [a.elapsed_time(b) for a, b in ev]


def bench_decode(torch, ops, workloads, steps, warmup, B=64, H=16, layers=24):
    """One decode step of a 24-layer stack at the 1.3B layer shape: 24
    in-place recurrent steps, one per layer state (24 x 64 MiB, so no layer
    finds its state in the 256 MB cache).  The 24 launches are captured once
    in a HIP graph and the graph is replayed, as a serving loop would run them;
    per-layer time = replay time / 24."""
    states = [torch.randn(B, H, 128, 128, device='cuda') for _ in range(layers)]
    x = workloads.make_inputs(B, 1, H, 128, 128, gate='scalar', dtype=torch.bfloat16, seed=4, device='cuda')

    def step_all():
        for i in range(layers):
            ops.fused_recurrent_gated_delta_rule(x.q, x.k, x.v, x.g, x.beta, initial_state=states[i],
                                                 inplace_final_state=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step_all()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step_all()
    total, ms = time_steps(torch, lambda i: graph.replay(), max(GRAPH_REPLAYS, steps), GRAPH_WARM_REPLAYS, 1)
    per_layer_ms = statistics.mean(ms) / layers
    byts = B * H * DECODE_BYTES_PER_SEQ_HEAD
    del graph, states
    return dict(avg_us=per_layer_ms * 1e3, GBs=byts / (per_layer_ms * 1e-3) / 1e9, bytes=byts)


def bench_generate(torch, workloads, reps=2):
    """The 1.3B-shape GDN language model (gdn_lm_1p3b: 24 layers, d2048, H16
    dk=dv=128, vocab 32000, bf16, random init): ragged prefill of its 64
    prompts (every prompt but its last token, one packed call per kernel),
    then 256 greedy decode steps for all 64 streams, each step (embedding,
    24 layers of projections, fused conv + recurrence + epilogue kernel and
    FFN, the tied head, the argmax) replayed from one HIP graph.  Host-clock
    timing around each phase, synchronised; the best of `reps` runs after a
    warm-up run that records the graph."""
    from vagus_amd.model import RaggedGenerator
    m, prompts, new = workloads.lm_workload('gdn_lm_1p3b')
    gen = RaggedGenerator(m)
    gen.prefill(prompts)
    gen.generate(4)
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        t0 = time.perf_counter()
        gen.prefill(prompts)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        toks = gen.generate(new)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if best is None or t2 - t0 < best[2] - best[0]:
            best = (t0, t1, t2)
    t0, t1, t2 = best
    c = m.config
    N = len(prompts)
    fed = sum(p.numel() - 1 for p in prompts)
    step_s = (t2 - t1) / new
    state_bytes = N * c['head_count'] * c['layer_count'] * DECODE_BYTES_PER_SEQ_HEAD
    weight_bytes = sum(p.numel() * p.element_size() for p in m.parameters())
    assert toks.shape == (N, new) and int(toks.min()) >= 0 and int(toks.max()) < c['vocab_size']
    del gen, m
    return {'workload': 'gdn_lm_1p3b: 24-layer GDN LM, d2048 H16 dk=dv=128, vocab 32000, bf16, random init, '
                        f'la_fused=True; {N} prompts U[64, 2048] ({fed + N} tokens), ragged prefill, {new} greedy steps',
            'prefill_ms': round((t1 - t0) * 1e3, 2), 'prefill_tok_s': round(fed / (t1 - t0), 1),
            'decode_ms': round((t2 - t1) * 1e3, 2), 'decode_step_ms': round(step_s * 1e3, 4),
            'gen_tok_s': round(N * new / (t2 - t1), 1),
            'decode_state_bytes_per_step': state_bytes, 'decode_weight_bytes_per_step': weight_bytes,
            'decode_state_GBs': round(state_bytes / step_s / 1e9, 1),
            'decode_total_GBs': round((state_bytes + weight_bytes) / step_s / 1e9, 1),
            'decode_total_frac_hbm': round((state_bytes + weight_bytes) / step_s / 1e9 / PEAK_HBM_GBS, 4),
            'end_to_end_s': round(t2 - t0, 4)}


def _settle(torch, fn, seconds):
    """Untimed calls of fn for `seconds` of host clock (synchronised every few calls)."""
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def _event_us(torch, fn, steps, warmup):
    """Mean event-timed microseconds of fn() over `steps` back-to-back calls,
    after LEG_SETTLE_S of untimed calls and `warmup` more."""
    _settle(torch, fn, LEG_SETTLE_S)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps * 1e3


def bench_layer_kernels(torch, ops, workloads, steps, warmup):
    """The layer's other kernels at the 340M shape (B8 T4096 H8 dk=dv=128):
    the short conv + SiLU over one projection (D = 1024, K = 4) and the
    RMSNorm x SiLU(gate) output epilogue, each over three rotating input
    copies, 24 calls replayed from a HIP graph; and the fused decode step (conv + SiLU with its caches, L2 norm,
    beta sigmoid, recurrence, epilogue) at the decode shape (B64 H16), 24
    rotating layers replayed from a HIP graph."""
    import torch.nn.functional as F
    g = torch.Generator(device='cpu').manual_seed(11)
    B, T, H, D, K = 8, 4096, 8, 128, 4

    def graph_us(fn, calls):
        # `calls` launches captured in one HIP graph and replayed: the kernels run back to
        # back, without the host's per-call time (longer than these kernels) between them
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(calls):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(calls):
                fn(i)
        _, ms = time_steps(torch, lambda i: graph.replay(), max(GRAPH_REPLAYS, steps), GRAPH_WARM_REPLAYS, 1)
        del graph
        return statistics.mean(ms) / calls * 1e3

    xs = [torch.randn(B, T, H * D, generator=g).bfloat16().cuda() for _ in range(3)]
    w = (0.5 * torch.randn(H * D, 1, K, generator=g)).cuda()
    # the weights in the module's dtype (a bf16 layer's ShortConv), and fp32 weights
    wb = w.bfloat16()
    conv_us = graph_us(lambda i: ops.causal_conv1d(xs[i % 3], wb, activation='silu'), 24)
    conv32_us = graph_us(lambda i: ops.causal_conv1d(xs[i % 3], w, activation='silu'), 24)
    conv_bytes = 2 * B * T * H * D * 2
    os_ = [torch.randn(B, T, H, D, generator=g).bfloat16().cuda() for _ in range(3)]
    gs = [torch.randn(B, T, H, D, generator=g).bfloat16().cuda() for _ in range(3)]
    gamma = (torch.rand(D, generator=g) + 0.5).bfloat16().cuda()
    ng_us = graph_us(lambda i: ops.rms_norm_gated(os_[i % 3], gs[i % 3], gamma), 24)
    ng_bytes = 3 * B * T * H * D * 2
    del xs, os_, gs
    # decode: every producer and the epilogue fused, 24 layers
    Bd, Hd, layers = 64, 16, 24
    Dd = Hd * D
    states = [torch.randn(Bd, Hd, D, D, generator=g).cuda() for _ in range(layers)]
    caches = [[torch.randn(Bd, K, Dd, generator=g).bfloat16().cuda() for _ in range(3)] for _ in range(layers)]
    cw = [(0.5 * torch.randn(Dd, 1, K, generator=g)).cuda() for _ in range(3)]
    qp, kp, vp = (torch.randn(Bd, 1, Dd, generator=g).bfloat16().cuda() for _ in range(3))
    gl = F.logsigmoid(torch.randn(Bd, 1, Hd, generator=g) + 4.0).cuda()
    bl = torch.randn(Bd, 1, Hd, generator=g).cuda()
    og = [torch.randn(Bd, 1, Hd, D, generator=g).bfloat16().cuda() for _ in range(layers)]

    def step_all():
        for i in range(layers):
            ops.hip_decode_step(qp, kp, vp, gl, bl, states[i], scale=D ** -0.5, conv_weights=cw,
                                conv_cache=caches[i], beta_logits=True, out_gate=og[i], out_norm_weight=gamma)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step_all()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step_all()
    _, ms = time_steps(torch, lambda i: graph.replay(), max(GRAPH_REPLAYS, steps), GRAPH_WARM_REPLAYS, 1)
    dec_us = statistics.mean(ms) / layers * 1e3
    # per (sequence, head): the plain step's bytes (state read and written, q k v o, g, beta), the three
    # conv caches read and written (K rows of the head's channels each), the epilogue gate row
    dec_bytes = Bd * Hd * (DECODE_BYTES_PER_SEQ_HEAD + 3 * 2 * K * D * 2 + D * 2)
    del graph, states, caches
    dec256_us, dec256_bytes = bench_decode_wide(torch, ops, steps, g)
    dec256b_us, dec256b_bytes = bench_decode_wide(torch, ops, steps, g, B=128)
    return {
        'short_conv': {'workload': 'causal_conv1d + SiLU, B8 T4096 D1024 K4 bf16, bf16 weights', 'us': round(conv_us, 2),
                       'achieved_GBs': round(conv_bytes / conv_us / 1e3, 1),
                       'frac_hbm': round(conv_bytes / conv_us / 1e3 / PEAK_HBM_GBS, 4),
                       'us_fp32_weights': round(conv32_us, 2),
                       'frac_hbm_fp32_weights': round(conv_bytes / conv32_us / 1e3 / PEAK_HBM_GBS, 4)},
        'output_epilogue': {'workload': 'rms_norm_gated, B8 T4096 H8 dv128 bf16', 'us': round(ng_us, 2),
                            'achieved_GBs': round(ng_bytes / ng_us / 1e3, 1),
                            'frac_hbm': round(ng_bytes / ng_us / 1e3 / PEAK_HBM_GBS, 4)},
        'decode_step_fused': {'workload': 'vgdr_decode_step (conv + caches, L2 norm, beta sigmoid, recurrence, '
                                          'epilogue) B64 H16 dk=dv=128 K4, 24 layers graph-replayed',
                              'us_per_step': round(dec_us, 2), 'achieved_GBs': round(dec_bytes / dec_us / 1e3, 1),
                              'frac_hbm': round(dec_bytes / dec_us / 1e3 / PEAK_HBM_GBS, 4)},
        'decode_step_fused_dv256': {
            'workload': 'vgdr_decode_step (conv + caches, L2 norm, beta sigmoid, KDA gate activation, recurrence, '
                        'epilogue) B64 H4 dk=128 dv=256 K4 (the dk 128 / dv 256 mixer heads), 24 layers graph-replayed',
            'us_per_step': round(dec256_us, 2), 'bytes_per_step': dec256_bytes,
            'achieved_GBs': round(dec256_bytes / dec256_us / 1e3, 1),
            'frac_hbm': round(dec256_bytes / dec256_us / 1e3 / PEAK_HBM_GBS, 4),
            'B128_us_per_step': round(dec256b_us, 2),
            'B128_frac_hbm': round(dec256b_bytes / dec256b_us / 1e3 / PEAK_HBM_GBS, 4)},
    }


def bench_decode_wide(torch, ops, steps, g, B=64, H=4, dk=128, dv=256, K=4, layers=24):
    """The one-kernel decode step at the dk 128 / dv 256 head shape (the
    reference's LAX1 / HAX mixers and its own layer bench): conv with its
    caches, L2 norm, beta sigmoid, the KDA gate activation, the recurrence
    and the epilogue, 24 rotating layers replayed from a HIP graph.  Returns
    (us per layer step, algorithmic bytes per step)."""
    import torch.nn.functional as F
    states = [torch.randn(B, H, dk, dv, generator=g).cuda() for _ in range(layers)]
    caches = [[torch.randn(B, K, H * d, generator=g).bfloat16().cuda() for d in (dk, dk, dv)] for _ in range(layers)]
    cw = [(0.5 * torch.randn(H * d, 1, K, generator=g)).bfloat16().cuda() for d in (dk, dk, dv)]
    qp, kp = (torch.randn(B, 1, H * dk, generator=g).bfloat16().cuda() for _ in range(2))
    vp = torch.randn(B, 1, H * dv, generator=g).bfloat16().cuda()
    f = torch.randn(B, 1, H, dk, generator=g).cuda()
    A_log = torch.rand(H, generator=g).cuda()
    dt_bias = torch.randn(H * dk, generator=g).cuda()
    bl = torch.randn(B, 1, H, generator=g).cuda()
    og = [torch.randn(B, 1, H, dv, generator=g).bfloat16().cuda() for _ in range(layers)]
    gamma = (torch.rand(dv, generator=g) + 0.5).bfloat16().cuda()

    def step_all():
        for i in range(layers):
            ops.hip_decode_step(qp, kp, vp, f, bl, states[i], scale=dk ** -0.5, conv_weights=cw,
                                conv_cache=caches[i], beta_logits=True, gate_in_kernel=True, A_log=A_log,
                                dt_bias=dt_bias, out_gate=og[i], out_norm_weight=gamma)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step_all()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step_all()
    _, ms = time_steps(torch, lambda i: graph.replay(), max(GRAPH_REPLAYS, steps), GRAPH_WARM_REPLAYS, 1)
    us = statistics.mean(ms) / layers * 1e3
    # per (sequence, head): the fp32 state read and written, q k (bf16, dk), v o (bf16, dv), the fp32 gate
    # pre-activation row (dk) and beta, the three conv caches read and written (K rows each), the gate row
    per = 2 * dk * dv * 4 + (2 * dk + 2 * dv) * 2 + dk * 4 + 4 + 2 * K * (2 * dk + dv) * 2 + dv * 2
    del graph, states, caches
    return us, B * H * per


def bench_backward(torch, ops, workloads, steps, warmup):
    """The chunked backward (vgdr_chunk_bwd through ops.chunk_gated_delta_rule_bwd)
    at the headline shape: gradients of o and the final state with respect to
    q, k, v, g, beta and the entry state, two rotating input copies."""
    g = torch.Generator(device='cpu').manual_seed(12)
    xs = [workloads.workload('gdn_340m', device='cuda') for _ in range(2)]
    dos = [torch.randn(*x.v.shape, generator=g).bfloat16().cuda() for x in xs]
    dST = torch.randn(*xs[0].initial_state.shape, generator=g).cuda()

    def step(i):
        x = xs[i % 2]
        ops.chunk_gated_delta_rule_bwd(x.q, x.k, x.v, x.g, x.beta, x.initial_state, dos[i % 2], dST,
                                       scale=DK ** -0.5)

    us = _event_us(torch, step, steps, warmup)

    # the training pair autograd runs for 16-bit inputs: the saving forward, then
    # the backward that reads the states and blocks it left
    def pair(i):
        x = xs[i % 2]
        o, S, ws = ops._chunk_fwd_saving(x.q, x.k, x.v, x.g, x.beta, x.initial_state, scale=DK ** -0.5,
                                         cu_seqlens=None, chunk_size=CHUNK)
        ops.chunk_gated_delta_rule_bwd(x.q, x.k, x.v, x.g, x.beta, x.initial_state, dos[i % 2], dST,
                                       scale=DK ** -0.5, saved_workspace=ws)

    pair_us = _event_us(torch, pair, steps, warmup)
    x0 = xs[0]
    th = x0.q.shape[0] * x0.q.shape[1] * x0.q.shape[2]
    del xs, dos
    tflops = th * 2 * FLOP_PER_TOKEN_HEAD / (us * 1e-6) / 1e12
    return {'workload': 'gdn_340m backward: dq, dk, dv, dg, dbeta, dh0 from do and dht, B8 T4096 H8 dk=dv=128 bf16',
            'kernels': 'chunk_prep_kernel + chunk_pipe_kernel (entry states only) + chunk_dhs_kernel + chunk_grad_kernel',
            'us': round(us, 1), 'tok_s': round(x0.q.shape[0] * x0.q.shape[1] / (us * 1e-6), 1),
            'flop_per_token_head': 2 * FLOP_PER_TOKEN_HEAD, 'achieved_tflops': round(tflops, 2),
            'frac_mfma': round(tflops / PEAK_BF16_TFLOPS, 5),
            'train_pair_us': round(pair_us, 1),
            'train_pair': 'vgdr_chunk_fwd_saving + vgdr_chunk_bwd_saved (what autograd runs for 16-bit inputs): '
                          'forward and backward with the entry states kept, not recomputed',
            'train_pair_tflops': round(th * 3 * FLOP_PER_TOKEN_HEAD / (pair_us * 1e-6) / 1e12, 2)}


def bench_kda_backward(torch, ops, workloads, steps, warmup, token_walk=True):
    """The KDA backward at the KDA prefill shape: gradients of o and the final
    state with respect to q, k, v, the per-channel g, beta and the entry state.
    The chunked backward (vgdr_chunk_bwd through
    ops.chunk_gated_delta_rule_bwd), the training pair autograd runs (saving
    forward + saved backward) and, for comparison, the token-walk backward
    (vgdr_scan_bwd through ops.scan_bwd)."""
    g = torch.Generator(device='cpu').manual_seed(13)
    x = workloads.workload('kda_prefill', device='cuda')
    do = torch.randn(*x.v.shape, generator=g).bfloat16().cuda()
    B, T, H = x.q.shape[:3]
    dST = torch.randn(B, H, x.q.shape[-1], x.v.shape[-1], generator=g).cuda()
    scale = DK ** -0.5

    def step(i):
        ops.chunk_gated_delta_rule_bwd(x.q, x.k, x.v, x.g, x.beta, x.initial_state, do, dST, scale=scale)

    us = _event_us(torch, step, steps, warmup)

    def pair(i):
        o, S, ws = ops._chunk_fwd_saving(x.q, x.k, x.v, x.g, x.beta, x.initial_state, scale=scale,
                                         cu_seqlens=None, chunk_size=CHUNK)
        ops.chunk_gated_delta_rule_bwd(x.q, x.k, x.v, x.g, x.beta, x.initial_state, do, dST, scale=scale,
                                       saved_workspace=ws)

    pair_us = _event_us(torch, pair, steps, warmup)
    # the plain recurrence (no delta rule, chunk_scan_vec(delta=False)) through the same kernels
    nodelta_us = _event_us(torch, lambda i: ops.chunk_gated_delta_rule_bwd(x.q, x.k, x.v, x.g, None, x.initial_state,
                                                                           do, dST, scale=scale, delta=False),
                           steps, warmup)
    # explicit write vectors (chunk_scan_vec(..., w=)) through the same kernels on chunk prep's WR blocks
    wv = (0.5 * torch.nn.functional.normalize(torch.randn(*x.q.shape, generator=g).cuda(), dim=-1)).to(x.q.dtype)
    w_us = _event_us(torch, lambda i: ops.chunk_write_bwd(x.q, x.k, x.v, wv, x.g, x.initial_state, do, dST,
                                                          scale=scale), steps, warmup)
    del wv
    # the reference's HAX1 / HAX2 training setting: chunk_kda with chunk_size=32 through autograd
    # (the per-channel backward runs 64-token chunks), forward and backward together
    leaves = [t.detach().clone().requires_grad_(True) for t in (x.q, x.k, x.v, x.g, x.beta)]

    def c32_pair(i):
        o, S = ops.chunk_kda(*leaves, scale=scale, initial_state=None, output_final_state=True, chunk_size=32)
        torch.autograd.backward([o, S], [do, dST])

    c32_us = _event_us(torch, c32_pair, steps, warmup)
    del leaves
    walk_us = None
    if token_walk:
        walk_us = _event_us(torch, lambda i: ops.scan_bwd(x.q, x.k, x.v, x.g, x.beta, x.initial_state, do, dST,
                                                          scale=scale), max(2, steps // 3), 1)
    th = B * T * H
    del x, do
    tflops = th * 2 * FLOP_PER_TOKEN_HEAD / (us * 1e-6) / 1e12
    r = {'workload': 'kda_prefill backward: dq, dk, dv, dg (per channel), dbeta, dh0 from do and dht, '
                     'B4 T8192 H8 dk=dv=128 bf16',
         'kernels': 'chunk_prep_kernel + chunk_pipe_kernel (entry states only) + chunk_dhs_kernel + chunk_grad_kernel '
                    '+ chunk_grad_vec_kernel',
         'us': round(us, 1), 'tok_s': round(B * T / (us * 1e-6), 1),
         'flop_per_token_head': 2 * FLOP_PER_TOKEN_HEAD, 'achieved_tflops': round(tflops, 2),
         'frac_mfma': round(tflops / PEAK_BF16_TFLOPS, 5),
         'train_pair_us': round(pair_us, 1),
         'train_pair': 'vgdr_chunk_fwd_saving + vgdr_chunk_bwd_saved (what autograd runs for 16-bit inputs)',
         'train_pair_tflops': round(th * 3 * FLOP_PER_TOKEN_HEAD / (pair_us * 1e-6) / 1e12, 2),
         'c32_autograd_pair_us': round(c32_us, 1),
         'c32_autograd_pair': 'chunk_kda(chunk_size=32) forward + autograd backward (the 64-token chunked backward)',
         'w_us': round(w_us, 1),
         'w': 'explicit write vectors (vgdr_chunk_bwd_w: the same kernels on chunk prep\'s WR blocks, dw for dbeta)',
         'nodelta_us': round(nodelta_us, 1),
         'nodelta': 'the recurrence without the delta rule (vgdr_chunk_bwd_nodelta: the same kernels on blocks '
                    'with TE = I and no K decay)'}
    if walk_us is not None:
        r['token_walk_us'] = round(walk_us, 1)
        r['token_walk'] = 'vgdr_scan_bwd (scan_walks_kernel + scan_grad_kernel + scan_bwd_finish_kernel)'
    return r


def cpu_baseline(torch, workloads):
    """The oracle's torch fp32 chunk form over the full headline workload."""
    from oracle import gdr
    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get('OMP_NUM_THREADS', '1024')))
    torch.set_num_threads(cores)
    x = workloads.workload('gdn_340m')
    q, k, v = x.q.float(), x.k.float(), x.v.float()

    def run():
        gdr.chunk_scalar(q, k, v, x.g, x.beta, x.initial_state, scale=128 ** -0.5, chunk_size=64)

    run()                                              # warmup
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    med = statistics.median(ts)
    tokens = q.shape[0] * q.shape[1]
    cpu = platform.processor() or platform.machine()
    try:
        with open('/proc/cpuinfo') as f:
            cpu = next(l.split(':', 1)[1].strip() for l in f if l.startswith('model name'))
    except Exception:
        pass
    return {'value': round(tokens / med, 1), 'unit': 'tok/s', 'cores': cores, 'kind': 'port',
            'sample': f'full gdn_340m workload (B8 T4096 H8 dk=dv=128, chunk 64), oracle.gdr.chunk_scalar '
                      f'in fp32, median of 3 after 1 warmup, {med:.2f} s per run, {cpu}'}


# kernel sources each measured traffic record depends on: a record whose
# fingerprint differs from the current sources is stale and is not reported
TRAFFIC_SOURCES = {
    'chunk_state': ('gdr_chunk.hip', 'gdr_chunk_layout.hpp', 'gdr_common.hpp', 'gdr_kernels.hpp'),
    'chunk_prep': ('gdr_chunk.hip', 'gdr_chunk_layout.hpp', 'gdr_common.hpp', 'gdr_kernels.hpp'),
    'recurrent': ('gdr_recurrent.hip', 'gdr_common.hpp', 'gdr_kernels.hpp'),
}
# (workload, kernel) -> substrings of the name rocprofv3 reports for it
# (demangled, or mangled where the demangler gives up on a __bf16 argument)
TRAFFIC_KERNELS = {
    ('gdn_340m', 'chunk_state'): ('vgdr::chunk_pipe_kernel<128, 64, 2,', 'chunk_pipe_kernelILi128ELi64ELi2E'),
    ('gdn_340m', 'chunk_prep'): ('vgdr::chunk_prep_kernel<128, 64,', 'chunk_prep_kernelILi128ELi64E'),
    ('decode_b64_h16', 'recurrent'): ('vgdr::recurrent_kernel<128, 128,', 'recurrent_kernelILi128ELi128E'),
}


def sources_sha(kernel):
    import hashlib
    h = hashlib.sha256()
    for name in TRAFFIC_SOURCES[kernel]:
        with open(os.path.join(ROOT, 'vagus_amd', 'csrc', name), 'rb') as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` ('chunk_state' / 'chunk_prep' / 'recurrent') on
    `workload`, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/traffic.json), or None when there is none or it was measured on
    other kernel sources."""
    path = os.path.join(ROOT, 'profiles', 'traffic.json')
    try:
        with open(path) as f:
            rec = json.load(f)[workload][kernel]
        if rec.get('sources_sha') != sources_sha(kernel):
            return None
        return int(rec['bytes_per_launch'])
    except (OSError, ValueError, KeyError, TypeError):
        return None


def write_traffic(run_dir):
    """profiles/traffic.json from rocprofv3 --pmc runs under run_dir: one
    counter_collection.csv per directory prefill_FETCH_SIZE, prefill_WRITE_SIZE
    (bench.py --prefill-only), decode_FETCH_SIZE, decode_WRITE_SIZE
    (--decode-only) and copy_FETCH_SIZE, copy_WRITE_SIZE (--calibrate-copy).
    Counters are in KiB per dispatch; a plain 1 GiB copy scales them to bytes."""
    import csv
    import glob

    def per_kernel(sub, counter):
        files = glob.glob(os.path.join(run_dir, f'{sub}_{counter}', '**', '*counter_collection.csv'), recursive=True)
        if not files:
            raise SystemExit(f'no counter_collection.csv under {run_dir}/{sub}_{counter}')
        vals = {}
        for row in csv.DictReader(open(files[0])):
            if row['Counter_Name'] == counter:
                vals.setdefault(row['Kernel_Name'], []).append(float(row['Counter_Value']))
        return {k: sum(v) / len(v) for k, v in vals.items()}

    def pick(table, names):
        hits = [v for k, v in table.items() if any(n in k for n in names)]
        if not hits:
            raise SystemExit(f'no kernel {names[0]} in the counters')
        return hits[0]

    copy_bytes = 1 << 30
    cf = max(per_kernel('copy', 'FETCH_SIZE').values())
    cw = max(per_kernel('copy', 'WRITE_SIZE').values())
    fs, ws = copy_bytes / 1024 / cf, copy_bytes / 1024 / cw
    out = {'calibration': {'copy_fetch_KiB': cf, 'copy_write_KiB': cw, 'fetch_scale': round(fs, 4),
                           'write_scale': round(ws, 4)}}
    for (wl, kern), names in TRAFFIC_KERNELS.items():
        sub = 'decode' if kern == 'recurrent' else 'prefill'
        f_kib = pick(per_kernel(sub, 'FETCH_SIZE'), names)
        w_kib = pick(per_kernel(sub, 'WRITE_SIZE'), names)
        rd, wr = f_kib * 1024 * fs, w_kib * 1024 * ws
        out.setdefault(wl, {})[kern] = {'bytes_per_launch': int(rd + wr), 'read_bytes': int(rd), 'write_bytes': int(wr),
                                        'fetch_KiB': f_kib, 'write_KiB': w_kib, 'kernel': names[0],
                                        'sources_sha': sources_sha(kern)}
    path = os.path.join(ROOT, 'profiles', 'traffic.json')
    with open(path, 'w') as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


# ---------------------------------------------------------------------------
# GEMM-phase MFMA utilisation (bench.py --gemm-phase): an instrumented copy of
# gdr_chunk.hip, built in a temporary directory from the current sources,
# stamps s_memtime around the state kernel's product stages for eight
# workgroups: the chain wave's P = K S stage (16 MFMAs, up to X), its TE X
# stage (6, up to the bf16 W), its state update (16, up to a read of S), and
# the first output wave's products (22 with 32-column tiles, 11 with 16).
# Empty asm statements pin each stage's operands after its first stamp and
# consume its results before its last, so the products cannot move across the
# stamps.  A stage's MFMA utilisation is (its MFMAs x 16 cycles) over its
# duration: at the bf16 peak (2.5 PFLOP/s over 1024 SIMDs at 2.4 GHz, 1017
# FLOP per SIMD-cycle) a 16x16x32 MFMA (16,384 FLOP) issues every 16 cycles;
# a calibration kernel's dependent chain (one MFMA per 15.9 cycles of the same
# counter) agrees.
# ---------------------------------------------------------------------------
PROBE_PATCHES = [
    ("namespace vgdr {", """namespace vgdr {
constexpr int GP_WG = 8, GP_STEPS = 128;
__device__ unsigned long long g_gp[GP_WG][GP_STEPS][8];
__device__ __forceinline__ int gp_slot(int b) {
    const int ids[GP_WG] = {0, 1, 37, 66, 101, 130, 199, 255};
#pragma unroll
    for (int i = 0; i < GP_WG; ++i) if (b == ids[i]) return i;
    return -1;
}
__device__ __forceinline__ unsigned long long gp_time() {
    __builtin_amdgcn_sched_barrier(0);
    const unsigned long long t = __builtin_amdgcn_s_memtime();
    __builtin_amdgcn_sched_barrier(0);
    return t;
}
__global__ void gp_calib_kernel(unsigned long long *out) {
    typedef __bf16 b8 __attribute__((ext_vector_type(8)));
    b8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(0.001f * (threadIdx.x + i)); b[i] = (__bf16)(0.002f * i); }
    f32x4 acc[8];
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{(float)j, 0.5f * j, 0.25f * j + threadIdx.x, 1.f + j};
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(acc[j]));
    const unsigned long long t0 = gp_time();
    asm volatile("" : "+v"(a), "+v"(b));
#pragma unroll
    for (int r = 0; r < 64; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
    float s = 0.f;
    for (int j = 0; j < 8; ++j) s += acc[j][0];
    asm volatile("" :: "v"(s));
    const unsigned long long t1 = gp_time();
    asm volatile("" : "+v"(a), "+v"(b));
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 64; ++r) d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, d, 0, 0, 0);
    asm volatile("" :: "v"(d[0]));
    const unsigned long long t2 = gp_time();
    if (threadIdx.x == 0) { out[0] = t1 - t0; out[1] = t2 - t1; }
}
}  // namespace vgdr
extern "C" int vgdr_probe_read(void *dst, long long n) {
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(vgdr::g_gp), (size_t)n, 0, hipMemcpyDeviceToHost);
}
extern "C" int vgdr_probe_clear() {
    static unsigned long long z[vgdr::GP_WG][vgdr::GP_STEPS][8];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(vgdr::g_gp), z, sizeof(z), 0, hipMemcpyHostToDevice);
}
extern "C" int vgdr_probe_calib(void *dst) {
    unsigned long long *d = nullptr;
    if (hipMalloc(&d, 16) != hipSuccess) return 1;
    hipLaunchKernelGGL(vgdr::gp_calib_kernel, dim3(1), dim3(64), 0, 0, d);
    hipError_t e = hipMemcpy(dst, d, 16, hipMemcpyDeviceToHost);
    hipFree(d);
    return (int)e;
}
namespace vgdr {"""),
    ("""            f32x4 U[NB];
            if constexpr (DELTA) {
                // P = K S (C layout), NB independent accumulation chains""", """            f32x4 U[NB];
            const int gps = gp_slot(blockIdx.x);
            unsigned long long gt0 = 0, gt1 = 0, gt2 = 0, gt3 = 0;
            gt0 = gp_time();
#pragma unroll
            for (int q = 0; q < NKB / 2; ++q) asm volatile("" : "+v"(Sb[q]));
            if constexpr (DELTA) {
                // P = K S (C layout), NB independent accumulation chains"""),
    ("""#pragma unroll
                for (int I = 0; I < NB; ++I) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};""", """#pragma unroll
                for (int q = 0; q < NB / 2; ++q) asm volatile("" :: "v"(Xb[q]));
                gt1 = gp_time();
#pragma unroll
                for (int q = 0; q < NB / 2; ++q) asm volatile("" : "+v"(Xb[q]));
#pragma unroll
                for (int I = 0; I < NB; ++I) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};"""),
    ("""            // S <- Gc S + (K*Gend)^T U~
            if constexpr (VEC) {""", """#pragma unroll
            for (int q = 0; q < NB / 2; ++q) asm volatile("" :: "v"(Wb[q]));
            gt2 = gp_time();
#pragma unroll
            for (int q = 0; q < NB / 2; ++q) asm volatile("" : "+v"(Wb[q]));
            // S <- Gc S + (K*Gend)^T U~
            if constexpr (VEC) {"""),
    ("""                                                    Ktr + (32 * q + 16) * PK + KQ::col(16 * kt)), Wb[q], S[kt]);
        }
        if (nchunks > 0) lds_barrier();                       // barrier n""", """                                                    Ktr + (32 * q + 16) * PK + KQ::col(16 * kt)), Wb[q], S[kt]);
            {
                float tmp = 0.f;
#pragma unroll
                for (int kt = 0; kt < NKB; ++kt) tmp += S[kt][0];
                asm volatile("" :: "v"(tmp));
            }
            gt3 = gp_time();
            if (gps >= 0 && wave == 0 && lane == 0 && c < GP_STEPS) {
                g_gp[gps][c][0] = gt0; g_gp[gps][c][1] = gt1; g_gp[gps][c][2] = gt2; g_gp[gps][c][3] = gt3;
            }
        }
        if (nchunks > 0) lds_barrier();                       // barrier n"""),
    ("""        unroll<NW>([&](auto s) { unroll<NR>([&](auto i) { ot[s][i] = f32x4{0.f, 0.f, 0.f, 0.f}; }); });""",
     """        unroll<NW>([&](auto s) { unroll<NR>([&](auto i) { ot[s][i] = f32x4{0.f, 0.f, 0.f, 0.f}; }); });
        const unsigned long long ot0 = gp_time();
#pragma unroll
        for (int s = 0; s < NW; ++s)
#pragma unroll
            for (int k = 0; k < NKB / 2; ++k) asm volatile("" : "+v"(Sn[s][k]));
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
            for (int k = 0; k < NKB / 2; ++k) asm volatile("" : "+v"(Qv[i][k]));"""),
    ("""        // the chunk's o rows as one buffer: rows past the sequence's end fall
        // outside it and their stores are dropped, with no lane-dependent branch""", """        {
            float tmp = 0.f;
            unroll<NW>([&](auto s) { unroll<NR>([&](auto i) { tmp += ot[s][i][0]; }); });
            asm volatile("" :: "v"(tmp));
        }
        const unsigned long long ot1 = gp_time();
        {
            const int gps = gp_slot(blockIdx.x);
            if (gps >= 0 && o == 0 && lane == 0 && c < GP_STEPS) { g_gp[gps][c][4] = ot0; g_gp[gps][c][5] = ot1; }
        }
        // the chunk's o rows as one buffer: rows past the sequence's end fall
        // outside it and their stores are dropped, with no lane-dependent branch"""),
    ("""    if (dtype == 1) {
        if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, __bf16) } VGDR_GATES(64, 64, __bf16) }""",
     """    if (dtype == 1 && dk == 128 && chunk == 64) { VGDR_GATES(128, 64, __bf16) }
    return hipErrorInvalidValue;
    if (dtype == 1) {
        if (dk == 64) { if (chunk == 32) { VGDR_GATES(64, 32, __bf16) } VGDR_GATES(64, 64, __bf16) }"""),
]


def build_phase_probe(outdir):
    """The instrumented library: gdr_chunk.hip with PROBE_PATCHES applied (each
    anchor must occur once in the current source), written to outdir beside
    copies of the headers, and the other sources as they are, compiled with
    the library's flags.  Returns the library path."""
    import concurrent.futures as cf
    import shutil
    import subprocess
    from vagus_amd import build as b
    os.makedirs(outdir, exist_ok=True)
    for f in os.listdir(b.CSRC):
        if f.endswith('.hpp'):
            shutil.copy(os.path.join(b.CSRC, f), os.path.join(outdir, f))
    path = os.path.join(outdir, 'gdr_chunk.hip')
    src = open(os.path.join(b.CSRC, 'gdr_chunk.hip')).read()
    for anchor, repl in PROBE_PATCHES:
        assert src.count(anchor) == 1, f'probe anchor not found once: {anchor[:60]!r}'
        src = src.replace(anchor, repl)
    open(path, 'w').write(src)
    # the instrumented file from outdir (beside the headers), every other file from the package
    srcs = [path] + [s for s in b.sources() if os.path.basename(s) != 'gdr_chunk.hip']
    objs = [os.path.join(outdir, os.path.basename(s)[:-4] + '.o') for s in srcs]

    def comp(so):
        r = subprocess.run([b.hipcc(), *b.HIPCC_FLAGS, '-c', so[0], '-o', so[1]], capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(r.stdout + r.stderr)
    with cf.ThreadPoolExecutor(len(srcs)) as ex:
        list(ex.map(comp, zip(srcs, objs)))
    lib = os.path.join(outdir, 'libphaseprobe.so')
    r = subprocess.run([b.hipcc(), f'--offload-arch={b.ARCH}', '-shared', '-fPIC', *objs, '-o', lib],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stdout + r.stderr)
    return lib


def gemm_phase(torch, workloads, lib_path, name):
    """Per-stage MFMA utilisation of the instrumented state kernel on `name`
    (gdn_340m or kda_prefill): stage medians in cycles of the s_memtime
    counter and the utilisation of every traced stage summed."""
    import ctypes
    import numpy as np
    from vagus_amd import _lib, ops
    lib = _lib.load(lib_path)
    for fn in ('vgdr_probe_read', 'vgdr_probe_calib'):
        getattr(lib, fn).argtypes = [ctypes.c_void_p, ctypes.c_longlong][:1 + (fn == 'vgdr_probe_read')]
    prev, _lib._lib = _lib._lib, lib
    try:
        xs = [workloads.workload(name, device='cuda') for _ in range(3)]
        gate = 'vector' if xs[0].g.dim() == 4 else 'scalar'

        def run(i, ev=None):
            x = xs[i % 3]
            return ops.chunk_scan(x.q, x.k, x.v, x.g, x.beta, gate=gate, delta=True, initial_state=x.initial_state,
                                  output_final_state=True, cu_seqlens=x.cu_seqlens, phase_event=ev)
        for i in range(200):
            run(i)
        torch.cuda.synchronize()
        cal = (ctypes.c_ulonglong * 2)()
        assert lib.vgdr_probe_calib(ctypes.addressof(cal)) == 0
        st = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(50)]
        for i in range(50):
            run(i, ev[i][0])
            ev[i][1].record(st)
        torch.cuda.synchronize()
        state_us = statistics.mean(a.elapsed_time(b) for a, b in ev) * 1e3
        lib.vgdr_probe_clear()
        run(0)
        torch.cuda.synchronize()
        buf = (ctypes.c_ulonglong * (8 * 128 * 8))()
        assert lib.vgdr_probe_read(ctypes.addressof(buf), ctypes.sizeof(buf)) == 0
    finally:
        _lib._lib = prev
    a = np.frombuffer(buf, dtype=np.uint64).reshape(8, 128, 8).astype(np.int64)
    nsteps = xs[0].q.shape[1] // CHUNK
    a = a[:, :nsteps]
    ok = (a[:, :, 0] > 0) & (a[:, :, 3] > a[:, :, 0]) & (a[:, :, 5] > a[:, :, 4])
    p_st, te_st = (a[:, :, 1] - a[:, :, 0])[ok], (a[:, :, 2] - a[:, :, 1])[ok]
    up_st, ch = (a[:, :, 3] - a[:, :, 2])[ok], (a[:, :, 3] - a[:, :, 0])[ok]
    out = (a[:, :, 5] - a[:, :, 4])[ok]
    step = np.diff(a[:, :, 0], axis=1)[:, 1:-1]
    n = int(ok.sum())
    n_chain, n_out = 38, (22 if gate == 'scalar' else 11)      # 32-column tiles (gdn_340m) or 16 (kda_prefill)
    c = 16.0
    frac = lambda m, d: round(m * c * n / float(d.sum()), 4)
    return {'workload': name, 'instrumented_state_us': round(state_us, 1), 'samples': n,
            'calib_cycles_independent_mfma': round(cal[0] / 512.0, 2), 'calib_cycles_dependent_mfma': round(cal[1] / 64.0, 2),
            'chain_step_cycles': float(np.median(step)),
            'chain_P_cycles': float(np.median(p_st)), 'chain_TE_cycles': float(np.median(te_st)),
            'chain_update_cycles': float(np.median(up_st)), 'output_cycles': float(np.median(out)),
            'chain_P_frac': frac(16, p_st), 'chain_TE_frac': frac(6, te_st), 'chain_update_frac': frac(16, up_st),
            'chain_frac': frac(n_chain, ch), 'output_frac': frac(n_out, out),
            'gemm_phase_frac': round((n_chain + n_out) * c * n / float(ch.sum() + out.sum()), 4),
            'chain_phase_share_of_step': round(float(np.median(ch)) / float(np.median(step)), 4)}


def measured_gemm_phase(workload):
    """The committed GEMM-phase record (profiles/gemm_phase.json) for workload,
    or None when it was measured on other kernel sources."""
    try:
        with open(os.path.join(ROOT, 'profiles', 'gemm_phase.json')) as f:
            rec = json.load(f)[workload]
        return rec if rec.get('sources_sha') == sources_sha('chunk_state') else None
    except (OSError, ValueError, KeyError, TypeError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=60)
    ap.add_argument('--warmup', type=int, default=100)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--settle', type=float, default=SETTLE_S, metavar='SECONDS',
                    help='clock-settle phase before the timed headline steps: back-to-back untimed prefill '
                         f'steps on the same inputs for this long (default {SETTLE_S}; reported as settle_s)')
    ap.add_argument('--prefill-only', nargs='?', const='gdn_340m', default=None, metavar='WORKLOAD',
                    help='only one prefill workload: gdn_340m (default, the headline line), kda_prefill or '
                         'gdn_varlen (for profiling)')
    ap.add_argument('--decode-only', action='store_true', help='only the decode step (for profiling)')
    ap.add_argument('--layer-only', action='store_true',
                    help='only the short conv, output epilogue and fused decode step (for profiling)')
    ap.add_argument('--backward-only', action='store_true', help='only the chunked backward (for profiling)')
    ap.add_argument('--generate-only', action='store_true',
                    help='only the 1.3B-shape LM generation (ragged prefill + 256 graph-replayed decode steps)')
    ap.add_argument('--calibrate-copy', action='store_true',
                    help='run only a plain 1 GiB device copy (x5): the reference point that scales '
                         'rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes')
    ap.add_argument('--gemm-phase', action='store_true',
                    help='build the instrumented state kernel (PROBE_PATCHES) and print the MFMA utilisation of its '
                         'product stages on gdn_340m and kda_prefill; with --write-gemm-phase also write '
                         'profiles/gemm_phase.json')
    ap.add_argument('--write-gemm-phase', action='store_true', help=argparse.SUPPRESS)
    ap.add_argument('--write-traffic', metavar='RUN_DIR',
                    help='write profiles/traffic.json from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs '
                         '(see write_traffic) and exit; needs no GPU')
    args = ap.parse_args()
    if args.write_traffic:
        write_traffic(args.write_traffic)
        return
    if args.gpus != 1:
        print(f'bench.py: measures one GPU only (the gated delta-rule core has no '
              f'cross-GPU path); --gpus {args.gpus} is not supported', file=sys.stderr)
        sys.exit(2)

    import torch
    from vagus_amd import ops, workloads

    assert torch.cuda.is_available(), 'bench.py needs a GPU'
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device='cuda')      # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'calibrate_copy_bytes': src.numel() * 4, 'launches': 5}), flush=True)
        return

    if args.gemm_phase:
        import tempfile
        lib = build_phase_probe(tempfile.mkdtemp(prefix='vgdr_probe_'))
        out = {}
        for name in ('gdn_340m', 'kda_prefill'):
            out[name] = dict(gemm_phase(torch, workloads, lib, name), sources_sha=sources_sha('chunk_state'))
            print(json.dumps(out[name]), flush=True)
        if args.write_gemm_phase:
            with open(os.path.join(ROOT, 'profiles', 'gemm_phase.json'), 'w') as f:
                json.dump(out, f, indent=1)
        return
    if args.generate_only:
        print(json.dumps(bench_generate(torch, workloads)), flush=True)
        return
    if args.backward_only:
        print(json.dumps(bench_backward(torch, ops, workloads, args.steps, args.warmup)), flush=True)
        print(json.dumps(bench_kda_backward(torch, ops, workloads, args.steps, args.warmup)),
              flush=True)
        return
    if args.layer_only:
        print(json.dumps(bench_layer_kernels(torch, ops, workloads, args.steps, args.warmup)), flush=True)
        return
    if args.decode_only:
        dec = bench_decode(torch, ops, workloads, args.steps, args.warmup)
        print(json.dumps({'decode_us_per_layer': round(dec['avg_us'], 2), 'achieved_GBs': round(dec['GBs'], 1)}),
              flush=True)
        return
    if args.prefill_only and args.prefill_only != 'gdn_340m':
        r = bench_prefill(torch, ops, workloads, args.prefill_only, args.steps, args.warmup)
        print(json.dumps({'workload': args.prefill_only, 'tok_s': round(r['tok_s'], 1),
                          'prep_ms': round(r['prep_ms'], 4), 'state_ms': round(r['state_ms'], 4),
                          'path_tflops': round(r['path_tflops'], 2), 'state_tflops': round(r['state_tflops'], 2)}),
              flush=True)
        return
    log(f'[bench] prefill gdn_340m (after {args.settle:.1f} s of clock settle on the same steps)')
    pre = bench_prefill(torch, ops, workloads, 'gdn_340m', args.steps, args.warmup, settle_s=args.settle)
    settle_s = pre['settle_s']
    extra = {}
    if not args.prefill_only:
        log('[bench] decode 1.3B layer shape')
        dec = bench_decode(torch, ops, workloads, args.steps, args.warmup)
        extra['decode'] = {'workload': 'gdn decode step B64 H16 dk=dv=128, 24 layer states, graph-replayed',
                           'us_per_step': round(dec['avg_us'], 2), 'achieved_GBs': round(dec['GBs'], 1),
                           'peak_GBs': PEAK_HBM_GBS, 'frac': round(dec['GBs'] / PEAK_HBM_GBS, 4),
                           'bytes_per_step': dec['bytes'],
                           'traffic': measured_traffic('decode_b64_h16', 'recurrent')}
        log('[bench] layer kernels: short conv, output epilogue, fused decode step')
        extra['layer_kernels'] = bench_layer_kernels(torch, ops, workloads, args.steps, args.warmup)
        log('[bench] backward gdn_340m')
        extra['backward'] = bench_backward(torch, ops, workloads, max(5, args.steps // 4), max(3, args.warmup // 10))
        log('[bench] backward kda_prefill')
        extra['kda_backward'] = bench_kda_backward(torch, ops, workloads, max(5, args.steps // 4), max(3, args.warmup // 10))
        log('[bench] generation gdn_lm_1p3b')
        extra['generation'] = bench_generate(torch, workloads)
        for name in ('kda_prefill', 'gdn_varlen'):
            log(f'[bench] prefill {name}')
            r = bench_prefill(torch, ops, workloads, name, max(3, args.steps // 3), max(2, args.warmup // 2),
                              settle_s=LEG_SETTLE_S)
            gpn = measured_gemm_phase(name)
            extra[name] = {'gemm_phase_frac': None if gpn is None else gpn['gemm_phase_frac'],
                           'tok_s': round(r['tok_s'], 1), 'op_ms': round(r['op_ms'], 4),
                           'prep_ms': round(r['prep_ms'], 4), 'state_ms': round(r['state_ms'], 4),
                           'path_tflops': round(r['path_tflops'], 2),
                           'path_frac_mfma': round(r['path_tflops'] / PEAK_BF16_TFLOPS, 5),
                           'state_tflops': round(r['state_tflops'], 2), 'tokens': r['tokens']}
    cpu = None
    if not args.no_cpu_baseline:
        log('[bench] cpu baseline')
        cpu = cpu_baseline(torch, workloads)

    tokens, H = pre['tokens'], pre['H']
    achieved = pre['state_tflops']
    gp = measured_gemm_phase('gdn_340m')
    state_gbs = tokens * H * STATE_BYTES_PER_TOKEN_HEAD / (pre['state_ms'] * 1e-3) / 1e9
    path_gbs = tokens * H * PREFILL_BYTES_PER_TOKEN_HEAD / (pre['op_ms'] * 1e-3) / 1e9
    line = {
        'metric': 'prefill tok/s + MFMA util; decode-step HBM GB/s vs peak (GDN/KDA, 1 GPU)',
        'value': round(pre['tok_s'], 1),
        'unit': 'tok/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'settle_s': round(settle_s, 3),
        'leg_settle_s': LEG_SETTLE_S,
        'ms_per_step': round(pre['total_s'] * 1e3 / args.steps, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic (seeded; q,k L2-normalised N(0,1), v N(0,1), beta sigmoid(N), g logsigmoid(N+4))',
        'config': {'workload': 'gdn_340m: GDN chunked prefill, 340M layer shape', 'B': 8, 'T': 4096,
                   'H': 8, 'dk': 128, 'dv': 128, 'chunk': 64, 'initial_state': '0.1*N(0,1)',
                   'tokens_per_step': tokens},
        'roofline': {'bound': 'mfma', 'achieved': round(achieved, 2), 'peak': PEAK_BF16_TFLOPS,
                     'unit': 'TFLOP/s', 'frac': round(achieved / PEAK_BF16_TFLOPS, 5),
                     'traffic': measured_traffic('gdn_340m', 'chunk_state'),
                     'kernel': 'chunk_pipe_kernel', 'kernel_avg_ms': round(pre['state_ms'], 4),
                     'flop_per_launch': tokens * H * STATE_FLOP_PER_TOKEN_HEAD,
                     'algorithmic_bytes_per_launch': tokens * H * STATE_BYTES_PER_TOKEN_HEAD,
                     'hbm_algorithmic_GBs': round(state_gbs, 1),
                     'gemm_phase_frac': None if gp is None else gp['gemm_phase_frac'],
                     'gemm_phase': None if gp is None else
                     {k: gp[k] for k in ('chain_frac', 'output_frac', 'chain_P_frac', 'chain_TE_frac',
                                         'chain_update_frac', 'chain_phase_share_of_step')},
                     'gemm_phase_method': 'MFMAs x 16 cycles over the s_memtime duration of the state kernel\'s '
                                          'product stages (chain P, TE X, update; output products) in an '
                                          'instrumented build (bench.py --gemm-phase, profiles/gemm_phase.json)'},
        'path': {'kernels': 'chunk_prep_kernel + chunk_pipe_kernel', 'op_ms': round(pre['op_ms'], 4),
                 'prep_ms': round(pre['prep_ms'], 4), 'state_ms': round(pre['state_ms'], 4),
                 'achieved_tflops': round(pre['path_tflops'], 2),
                 'frac_mfma': round(pre['path_tflops'] / PEAK_BF16_TFLOPS, 5),
                 'flop_per_token_head': FLOP_PER_TOKEN_HEAD, 'hbm_algorithmic_GBs': round(path_gbs, 1),
                 'prep_traffic': measured_traffic('gdn_340m', 'chunk_prep')},
        'cpu_baseline': cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
