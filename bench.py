#!/usr/bin/env python3
"""Benchmark of the teeny-kernels hot path on one MI355X.

Default workload (the norm + activation chain, bf16 in/out, fp32 stats):
X[16384, 4096] ~ N(0,1); one step is
    Y1 = LayerNorm(X)  (eps 1e-5, gamma ~ N(1, .02), beta ~ N(0, .02))
    G1 = GELU-tanh(Y1);  S1 = SiLU(Y1)
    Y2 = RMSNorm(X)    (eps 1e-8, gamma ~ N(1, .02))
    G2 = GELU-tanh(Y2);  S2 = SiLU(Y2)
six HBM-bound kernels, each moving 2 x 128 MiB.  `value` is the step's
algorithmic bytes / step time in GB/s.  Inputs are resident in HBM before
the timed region; every kernel of the timed steps is bracketed by HIP events
on the launch stream, which gives each kernel's average duration for the
roofline object.

Other workloads (--workload): attention_causal_s2048, attention_s4096,
resnet50_convs, w8a16_gemm, w8a16_conv, conv2d_f32 — TFLOP/s lines.

The cpu_baseline object times the CPU oracle (a C restatement of the
reference kernels, oracle/) on the host, on the workload stated in its
`sample` field.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GB/s or TFLOP/s per op vs MI355X roofline; speedup vs host-CPU teenygrad path"
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2500.0    # dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3     # fp32 vector


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_threads():
    env = os.environ.get("TEENY_CPU_THREADS")
    if env:
        return int(env)
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))  # the GPU box's CPU share is 16 threads


class Timer:
    """Per-kernel HIP events on the launch stream.  Events are created before
    the timed pass so that recording one costs only the enqueue."""

    def __init__(self, tg, stream, kernels_per_step, steps):
        self.stream = stream
        self.pool = [tg.Event() for _ in range(2 * kernels_per_step * steps)]
        self.used = 0
        self.pairs = {}

    def run(self, name, fn):
        a, b = self.pool[self.used], self.pool[self.used + 1]
        self.used += 2
        a.record(self.stream)
        fn()
        b.record(self.stream)
        self.pairs.setdefault(name, []).append((a, b))

    def avg_ms(self):
        return {k: float(np.mean([a.elapsed_ms(b) for a, b in v])) for k, v in self.pairs.items()}


def timed_steps(tg, dev, stream, step, steps, warmup, kernels_per_step):
    """Warmup, then two timed passes of `steps` steps each:
    pass 1 (the reported step time) launches the kernels back to back between
    two events; pass 2 brackets every kernel with its own event pair for the
    per-kernel durations (the event markers add small gaps between kernels,
    which is why pass 1 alone gives the step time)."""
    for _ in range(warmup):
        step(None)
    dev.synchronize()
    t0, t1 = tg.Event(), tg.Event()
    t0.record(stream)
    wall0 = time.perf_counter()
    for _ in range(steps):
        step(None)
    t1.record(stream)
    t1.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_ms(t1) / steps
    timer = Timer(tg, stream, kernels_per_step, steps)
    dev.synchronize()
    for _ in range(steps):
        step(timer)
    dev.synchronize()
    return ms, wall, timer.avg_ms()


def launch(timer, name, fn):
    if timer is None:
        fn()
    else:
        timer.run(name, fn)


def load_traffic(workload):
    """HBM bytes per launch of the dominant kernel from the committed rocprof
    counter summary (profiles/<workload>_traffic.json), or None."""
    p = os.path.join(ROOT, "profiles", f"{workload}_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("traffic_bytes_per_launch")


# ── default: norm + activation chain ────────────────────────────────────────

NORM_M, NORM_N = 16384, 4096


def norm_inputs():
    from teenygrad_amd import synthetic
    from teenygrad_amd.dtypes import round_bf16
    x = round_bf16(synthetic.normal(synthetic.workload_seed(1, 0), (NORM_M, NORM_N)))
    g1 = round_bf16(synthetic.normal(synthetic.workload_seed(1, 1), (NORM_N,), 1.0, 0.02))
    b1 = round_bf16(synthetic.normal(synthetic.workload_seed(1, 2), (NORM_N,), 0.0, 0.02))
    g2 = round_bf16(synthetic.normal(synthetic.workload_seed(1, 3), (NORM_N,), 1.0, 0.02))
    return x, g1, b1, g2


def bench_norm_act(args, tg, dev, stream):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import to_bf16
    x, g1, b1, g2 = norm_inputs()
    up = lambda a: dev.upload(to_bf16(a), tg.bf16)
    xb, g1b, b1b, g2b = up(x), up(g1), up(b1), up(g2)
    shape = (NORM_M, NORM_N)
    y1, gl, sl, y2, gr, sr = (tg.Buffer(tg.bf16, shape) for _ in range(6))
    rrms = tg.Buffer(tg.f32, (NORM_M,))
    elem = NORM_M * NORM_N
    io = 2 * elem * 2  # read X + write Y, bf16
    bytes_of = {"layer_norm": io + 2 * NORM_N * 2, "gelu(ln)": io, "silu(ln)": io,
                "rms_norm": io + NORM_N * 2 + NORM_M * 4, "gelu(rms)": io, "silu(rms)": io}

    def step(t):
        launch(t, "layer_norm", lambda: K.layer_norm(xb, g1b, b1b, 1e-5, y=y1, stream=stream))
        launch(t, "gelu(ln)", lambda: K.gelu(y1, y=gl, stream=stream))
        launch(t, "silu(ln)", lambda: K.silu(y1, y=sl, stream=stream))
        launch(t, "rms_norm", lambda: K.rms_norm(xb, g2b, 1e-8, y=y2, rrms=rrms, stream=stream))
        launch(t, "gelu(rms)", lambda: K.gelu(y2, y=gr, stream=stream))
        launch(t, "silu(rms)", lambda: K.silu(y2, y=sr, stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, 6)
    step_bytes = sum(bytes_of.values())
    value = step_bytes / (ms * 1e-3) / 1e9
    dom = max(per, key=per.get)
    achieved = bytes_of[dom] / (per[dom] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": load_traffic("norm_act"), "algorithmic_bytes": bytes_of[dom],
            "avg_us": round(per[dom] * 1e3, 2)}
    ops = {k: {"us": round(v * 1e3, 2), "GB/s": round(bytes_of[k] / (v * 1e-3) / 1e9, 1),
               "frac": round(bytes_of[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)} for k, v in per.items()}

    cpu = None
    if not args.no_cpu:
        import oracle
        th = cpu_threads()
        oracle.set_threads(th)
        times = []
        for _ in range(3):
            c0 = time.perf_counter()
            ln = oracle.layer_norm(x, g1, b1, 1e-5)
            oracle.gelu(ln)
            oracle.silu(ln)
            rm, _ = oracle.rms_norm(x, g2, 1e-8)
            oracle.gelu(rm)
            oracle.silu(rm)
            times.append(time.perf_counter() - c0)
        cs = float(np.median(times))
        cpu = {"value": round(step_bytes / cs / 1e9, 2), "unit": "GB/s", "cores": th, "kind": "port",
               "seconds_per_step": round(cs, 3),
               "sample": "the full step (6 ops on [16384, 4096]) in fp32 on the bf16-rounded "
                         "inputs, median of 3 runs; bytes counted as bf16 like the GPU line"}
    return {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms, 4),
        "dtype": "bf16", "scaling": "weak",
        "config": {"workload": "norm_act_chain: X[16384,4096] bf16 -> LayerNorm -> GELU-tanh, SiLU; "
                               "RMSNorm -> GELU-tanh, SiLU (fp32 stats)",
                   "M": NORM_M, "N": NORM_N, "ops_per_step": 6, "bytes_per_step": step_bytes},
        "roofline": roof, "cpu_baseline": cpu, "ops": ops, "wall_s": round(wall, 3),
    }


# ── attention ───────────────────────────────────────────────────────────────


def bench_act_backward(args, tg, dev, stream):
    """Activation gradients on the norm workload's shape: dy and the saved tensor in, dx out
    (relu takes the forward output, gelu/silu the forward input); 3 x 128 MiB per op."""
    from teenygrad_amd import kernels as K
    from teenygrad_amd import synthetic
    from teenygrad_amd.dtypes import round_bf16, to_bf16
    x, _, _, _ = norm_inputs()
    dy = round_bf16(synthetic.normal(synthetic.workload_seed(1, 4), (NORM_M, NORM_N)))
    y = np.maximum(x, 0)
    up = lambda a: dev.upload(to_bf16(a), tg.bf16)
    xb, yb, dyb = up(x), up(y), up(dy)
    shape = (NORM_M, NORM_N)
    dr, dg, ds = (tg.Buffer(tg.bf16, shape) for _ in range(3))
    io = 3 * NORM_M * NORM_N * 2  # read dy + saved, write dx, bf16
    bytes_of = {"relu_backward": io, "gelu_backward": io, "silu_backward": io}

    def step(t):
        launch(t, "relu_backward", lambda: K.relu_backward(dyb, yb, dx=dr, stream=stream))
        launch(t, "gelu_backward", lambda: K.gelu_backward(dyb, xb, dx=dg, stream=stream))
        launch(t, "silu_backward", lambda: K.silu_backward(dyb, xb, dx=ds, stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, 3)
    step_bytes = sum(bytes_of.values())
    dom = max(per, key=per.get)
    achieved = bytes_of[dom] / (per[dom] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": load_traffic("act_backward"), "algorithmic_bytes": bytes_of[dom],
            "avg_us": round(per[dom] * 1e3, 2)}
    ops = {k: {"us": round(v * 1e3, 2), "GB/s": round(bytes_of[k] / (v * 1e-3) / 1e9, 1),
               "frac": round(bytes_of[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)} for k, v in per.items()}
    cpu = None
    if not args.no_cpu:
        import oracle
        th = cpu_threads()
        oracle.set_threads(th)
        times = []
        for _ in range(3):
            c0 = time.perf_counter()
            oracle.relu_backward(dy, y)
            oracle.gelu_backward(dy, x)
            oracle.silu_backward(dy, x)
            times.append(time.perf_counter() - c0)
        cs = float(np.median(times))
        cpu = {"value": round(step_bytes / cs / 1e9, 2), "unit": "GB/s", "cores": th, "kind": "port",
               "seconds_per_step": round(cs, 3),
               "sample": "the full step (3 gradients on [16384, 4096]) in fp32 on the bf16-rounded "
                         "inputs, median of 3 runs; bytes counted as bf16 like the GPU line"}
    return {
        "metric": METRIC, "value": round(step_bytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
        "ms_per_step": round(ms, 4), "dtype": "bf16", "scaling": "weak",
        "config": {"workload": "activation gradients: dy, x|y [16384,4096] bf16 -> dx for "
                               "ReLU, GELU-tanh, SiLU (fp32 math)",
                   "M": NORM_M, "N": NORM_N, "ops_per_step": 3, "bytes_per_step": step_bytes},
        "roofline": roof, "cpu_baseline": cpu, "ops": ops, "wall_s": round(wall, 3),
    }


def bench_attention(args, tg, dev, stream, s, causal, idx):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import to_bf16
    bh, d = 256, 128
    rng = np.random.default_rng(0x7EE70000 + idx)
    q, k, v = (dev.upload(to_bf16(rng.standard_normal((bh, s, d), dtype=np.float32)), tg.bf16)
               for _ in range(3))
    o = tg.Buffer(tg.bf16, (bh, s, d))
    lse = tg.Buffer(tg.f32, (bh, s))
    flops = 4.0 * bh * s * s * d * (0.5 if causal else 1.0)
    name = "flash_attention_bf16"

    def step(t):
        launch(t, name, lambda: K.flash_attention(q, k, v, None, causal, o=o, lse=lse, stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, 1)
    tf = flops / (ms * 1e-3) / 1e12
    ach = flops / (per[name] * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu:
        import oracle
        th = cpu_threads()
        oracle.set_threads(th)
        # sample: every query row of the first (batch, head) pair — programs
        # [0, S) of the oracle's (bh, row) grid; all heads cost the same, so the
        # full workload is BH times the sample
        qh = np.random.default_rng(1).standard_normal((1, s, d), dtype=np.float32)
        c0 = time.perf_counter()
        oracle.flash_attention(qh, qh, qh, None, causal)
        cs = time.perf_counter() - c0
        full = cs * bh
        cpu = {"value": round(flops / full / 1e12, 5), "unit": "TFLOP/s", "cores": th, "kind": "port",
               "sample": f"one (batch, head) of {bh}: all {s} query rows in the fp32 oracle, "
                         f"{cs:.2f} s, scaled x{bh}", "extrapolated_seconds": round(full, 1)}
    return {"metric": METRIC, "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "dtype": "bf16", "scaling": "weak",
            "config": {"workload": f"sdpa {'causal' if causal else 'non-causal'} bf16 B*H=256 S={s} D=128",
                       "flop_per_step": flops},
            "roofline": {"bound": "mfma", "kernel": name, "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                         "traffic": load_traffic(args.workload),
                         "algorithmic_bytes": 4 * bh * s * d * 2 + bh * s * 4,
                         "avg_us": round(per[name] * 1e3, 2)},
            "cpu_baseline": cpu, "wall_s": round(wall, 3)}


# ── ResNet-50 conv stack ────────────────────────────────────────────────────


def resnet50_convs():
    """(name, Cin, Cout, H_in, K, stride, pad, relu) for the 53 convs, batch 64, 224x224."""
    layers = [("stem", 3, 64, 224, 7, 2, 3, True)]
    cfg = [(64, 256, 3, 56), (128, 512, 4, 56), (256, 1024, 6, 28), (512, 2048, 3, 14)]
    cin = 64
    for li, (w, out, blocks, hin) in enumerate(cfg):
        s = 1 if li == 0 else 2
        for bi in range(blocks):
            h = hin if bi == 0 else (hin // s)
            stride = s if bi == 0 else 1
            layers.append((f"l{li + 1}b{bi}c1", cin, w, h, 1, 1, 0, True))
            layers.append((f"l{li + 1}b{bi}c2", w, w, h, 3, stride, 1, True))
            h2 = h // stride
            layers.append((f"l{li + 1}b{bi}c3", w, out, h2, 1, 1, 0, False))
            if bi == 0:
                layers.append((f"l{li + 1}b{bi}ds", cin, out, h, 1, stride, 0, False))
            cin = out
    return layers


def attach_workspace(tg, dev, stream, sizes):
    """Gives the stream one caller-owned scratch buffer big enough for every
    op of the workload (split-K partials, space-to-depth copies); returns
    its size.  Allocated before timing, as an executor would."""
    need = max(list(sizes) + [0])
    if need > 0:
        stream.set_workspace(dev.buffer(tg.i8, (need,)))
    return need


def bench_resnet(args, tg, dev, stream):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import to_bf16
    B = 64
    rng = np.random.default_rng(0x7EE70003)
    layers = resnet50_convs()
    assert len(layers) == 53
    bufs = []
    flops = 0.0
    total_bytes = 0
    for name, cin, cout, h, k, s, p, relu in layers:
        oh = (h + 2 * p - k) // s + 1
        x = dev.upload(to_bf16(rng.random((B, h, h, cin), dtype=np.float32)), tg.bf16)
        w = dev.upload(to_bf16((rng.standard_normal((cout, k, k, cin), dtype=np.float32)
                                * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)), tg.bf16)
        b = dev.upload(to_bf16(rng.normal(0, 0.01, cout).astype(np.float32)), tg.bf16)
        y = tg.Buffer(tg.bf16, (B, oh, oh, cout))
        f = 2.0 * B * oh * oh * cout * cin * k * k
        flops += f
        total_bytes += 2 * (B * h * h * cin + cout * k * k * cin + cout + B * oh * oh * cout)
        bufs.append((name, x, w, b, y, s, p, relu, f))
    ws = attach_workspace(tg, dev, stream, (
        K.conv2d_workspace_size((B, h, h, cin), (cout, k, k, cin), s, p, 1, tg.bf16, "nhwc")
        for name, cin, cout, h, k, s, p, relu in layers))
    log(f"[bench] stream workspace {ws / 2**20:.1f} MiB")

    def step(t):
        for name, x, w, b, y, s, p, relu, _ in bufs:
            launch(t, name, lambda: K.conv2d(x, w, b, s, p, 1, "relu" if relu else None, "nhwc", y=y,
                                             stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, len(bufs))
    tf = flops / (ms * 1e-3) / 1e12
    by_layer = {}
    for bb in bufs:
        n, f = bb[0], bb[-1]
        by_layer[n] = {"us": round(per[n] * 1e3, 1), "TFLOP/s": round(f / (per[n] * 1e-3) / 1e12, 1)}
    dom = max(per, key=per.get)
    fdom = [bb[-1] for bb in bufs if bb[0] == dom][0]
    ach = fdom / (per[dom] * 1e-3) / 1e12
    return {"metric": METRIC, "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "dtype": "bf16", "scaling": "weak",
            "config": {"workload": "resnet50 53 convs bf16 NHWC batch 64 224x224, BN folded to bias, ReLU fused",
                       "flop_per_step": flops, "bytes_per_step": total_bytes},
            "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": None},
            "layers": by_layer, "cpu_baseline": None, "wall_s": round(wall, 3)}


# ── W8A16 ───────────────────────────────────────────────────────────────────


def bench_w8a16(args, tg, dev, stream):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import to_bf16
    m = 4096
    rng = np.random.default_rng(0x7EE70005)
    problems = []
    for k, n in ((4096, 11008), (11008, 4096)):
        x = dev.upload(to_bf16(rng.standard_normal((m, k), dtype=np.float32)), tg.bf16)
        wf = dev.upload(rng.normal(0, 0.02, (n, k)).astype(np.float32))
        q, s, _, _ = K.quantize_affine(wf, [n, k], "channel", 0)
        del wf
        y = tg.Buffer(tg.bf16, (m, n))
        problems.append((f"w8a16 {m}x{k}->{n}", x, q, s, y, 2 * m * k + n * k + 4 * n + 2 * m * n, 2.0 * m * n * k))
    attach_workspace(tg, dev, stream, (K.linear_workspace_size(m, n, k, tg.i8)
                                       for k, n in ((4096, 11008), (11008, 4096))))

    def step(t):
        for name, x, q, s, y, _, _ in problems:
            launch(t, name, lambda: K.w8a16_linear(x, q, s, y=y, stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, len(problems))
    flops = sum(p[-1] for p in problems)
    tf = flops / (ms * 1e-3) / 1e12
    ops = {p[0]: {"us": round(per[p[0]] * 1e3, 1), "TFLOP/s": round(p[-1] / (per[p[0]] * 1e-3) / 1e12, 1)}
           for p in problems}
    dom = max(per, key=per.get)
    fdom = [p[-1] for p in problems if p[0] == dom][0]
    dom_bytes = [p[-2] for p in problems if p[0] == dom][0]  # x bf16 + int8 q + fp32 scales + y bf16
    ach = fdom / (per[dom] * 1e-3) / 1e12
    return {"metric": METRIC, "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "dtype": "bf16", "scaling": "weak",
            "config": {"workload": "w8a16 GEMMs M=4096: K=4096->N=11008 and K=11008->N=4096, int8 per-channel weights",
                       "flop_per_step": flops},
            "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                         "traffic": load_traffic(args.workload), "algorithmic_bytes": dom_bytes},
            "ops": ops, "cpu_baseline": None, "wall_s": round(wall, 3)}


def bench_w8a16_conv(args, tg, dev, stream):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import to_bf16
    B, C, H = 32, 256, 28
    rng = np.random.default_rng(0x7EE70006)
    x = dev.upload(to_bf16(rng.standard_normal((B, H, H, C), dtype=np.float32)), tg.bf16)
    wf = dev.upload(rng.normal(0, 0.02, (C, 3, 3, C)).astype(np.float32))
    q, s, _, _ = K.quantize_affine(wf, [C, 3, 3, C], "channel", 0)
    y = tg.Buffer(tg.bf16, (B, H, H, C))
    flops = 2.0 * B * H * H * C * C * 9
    name = "w8a16_conv3x3"
    attach_workspace(tg, dev, stream, [K.conv2d_workspace_size((B, H, H, C), (C, 3, 3, C), 1, 1, 1, tg.i8)])

    def step(t):
        launch(t, name, lambda: K.w8a16_conv2d(x, q, s, None, 1, 1, y=y, stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, 1)
    ach = flops / (per[name] * 1e-3) / 1e12
    return {"metric": METRIC, "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
            "ms_per_step": round(ms, 4), "dtype": "bf16", "scaling": "weak",
            "config": {"workload": "w8a16 conv3x3 NHWC 32x256x28x28 -> 256, p1", "flop_per_step": flops},
            "roofline": {"bound": "mfma", "kernel": name, "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": None},
            "cpu_baseline": None, "wall_s": round(wall, 3)}


def bench_conv_f32(args, tg, dev, stream):
    from teenygrad_amd import kernels as K
    rng = np.random.default_rng(0x7EE70000)
    x = rng.standard_normal((1, 64, 56, 56), dtype=np.float32)
    w = (rng.standard_normal((64, 64, 3, 3), dtype=np.float32) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = (rng.standard_normal(64, dtype=np.float32) * 0.01).astype(np.float32)
    xb, wb, bb = dev.upload(x), dev.upload(w), dev.upload(b)
    y = tg.Buffer(tg.f32, (1, 64, 56, 56))
    flops = 2.0 * 64 * 56 * 56 * 64 * 9
    name = "conv2d_bias_relu_f32"

    def step(t):
        launch(t, name, lambda: K.conv2d(xb, wb, bb, 1, 1, 1, "relu", y=y, stream=stream))

    ms, wall, per = timed_steps(tg, dev, stream, step, args.steps, args.warmup, 1)
    ach = flops / (per[name] * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu:
        import oracle
        th = cpu_threads()
        oracle.set_threads(th)
        times = []
        for _ in range(3):
            c0 = time.perf_counter()
            oracle.relu(oracle.conv2d_nchw(x, w, b, padding=1))
            times.append(time.perf_counter() - c0)
        cs = float(np.median(times))
        cpu = {"value": round(flops / cs / 1e12, 4), "unit": "TFLOP/s", "cores": th, "kind": "port",
               "sample": "the full conv (+bias) and ReLU, median of 3"}
    return {"metric": METRIC, "value": round(flops / (ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(ms, 4), "dtype": "f32", "scaling": "weak",
            "config": {"workload": "conv2d+bias+relu fp32 NCHW 1x64x56x56 -> 64, 3x3 s1 p1", "flop_per_step": flops},
            "roofline": {"bound": "mfma", "kernel": name, "achieved": round(ach, 3), "peak": FP32_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / FP32_PEAK_TFLOPS, 4), "traffic": None},
            "cpu_baseline": cpu, "wall_s": round(wall, 3)}


WORKLOADS = {
    "norm_act": bench_norm_act,
    "act_backward": bench_act_backward,
    "attention_causal_s2048": lambda a, tg, d, s: bench_attention(a, tg, d, s, 2048, True, 2),
    "attention_s4096": lambda a, tg, d, s: bench_attention(a, tg, d, s, 4096, False, 2),
    "resnet50_convs": bench_resnet,
    "w8a16_gemm": bench_w8a16,
    "w8a16_conv": bench_w8a16_conv,
    "conv2d_f32": bench_conv_f32,
}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="norm_act", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="first run one device-to-device copy of BYTES (a reference kernel of known "
                         "traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the hot path has no multi-GPU component in this build "
              f"(--gpus {args.gpus} requested); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import teenygrad_amd as tg

    dev = tg.open(int(os.environ.get("LOCAL_RANK", "0")))
    stream = tg.Stream.create()
    log(f"[bench] {args.workload} steps={args.steps} warmup={args.warmup} on {dev.info()['arch']}")
    if args.copy_calibration:
        src, dst = tg.Buffer(tg.i8, (args.copy_calibration,)), tg.Buffer(tg.i8, (args.copy_calibration,))
        src.zero_(stream)
        tg.check(tg._lib.lib.teeny_hip_memcpy_d2d(dst.ptr, src.ptr, args.copy_calibration, stream.handle))
        stream.synchronize()
        del src, dst
    res = WORKLOADS[args.workload](args, tg, dev, stream)
    line = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"),
            "higher_is_better": True, "scaling": res.pop("scaling"), "vs_baseline": None,
            "dtype": res.pop("dtype"), "data": "synthetic (seeded N(0,1) inputs, random-init params)"}
    line.update(res)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
