#!/usr/bin/env python3
"""Benchmark of the teeny-kernels hot path on one MI355X.

The default run measures all five configurations and prints one JSON line.
Its headline `value` is configuration 2, the norm + activation chain (bf16
in/out, fp32 stats): X[16384, 4096] ~ N(0,1); one step is
    Y1 = LayerNorm(X)  (eps 1e-5, gamma ~ N(1, .02), beta ~ N(0, .02))
    G1 = GELU-tanh(Y1);  S1 = SiLU(Y1)
    Y2 = RMSNorm(X)    (eps 1e-8, gamma ~ N(1, .02))
    G2 = GELU-tanh(Y2);  S2 = SiLU(Y2)
six HBM-bound kernels, each moving 2 x 128 MiB; `value` is the step's
algorithmic bytes / step time in GB/s.  The `configs` object carries one
entry per configuration (1: conv2d+bias+ReLU fp32 NCHW; 2: the chain above;
3: causal SDPA S=2048 and non-causal S=4096; 4: the 53 ResNet-50 convs at
batch 64; 5: the two W8A16 GEMMs and the int8 3x3 conv), each with its own
roofline object (dominant kernel) and CPU baseline.

Inputs are resident in HBM before any timed region.  Each workload runs W
warmup steps eagerly, then more eager steps for at least WARM_MS (60 ms,
--warm-ms) of wall time, then K steps captured into one HIP graph, replayed
once untimed and once between two HIP events on the launch stream (the step
time).  The time-based warm-up is there for the clock: under load the
MI355X raises its shader clock over tens of milliseconds (measured with
s_memtime against s_memrealtime in a causal attention kernel: 1.45 GHz
after 4 ms of back-to-back launches, 1.64 GHz after 13 ms, a settled
1.78-1.81 GHz from 40 ms on), so a short op timed right after a few
launches would be timed on the ramp.  Then every op of the step is captured
K times over into a graph of its own and timed the same way after 10 ms of
its own eager launches (its average launch duration, used by the roofline
objects).  Graph replay keeps Python's launch overhead out of the GPU's
timeline, as an executor's captured graph would.  Ops whose buffers would fit the 256 MB Infinity Cache
cycle through 2-4 device copies of their operands, so that repeated launches
read HBM rather than the previous launch's cached bytes.

The CPU baselines time the oracle (oracle/, a C restatement of the reference
kernels' program grids and loops, rebuilt here with -march=native) on this
host's cores: the median of repeated runs after one warm-up (at least 3, and
as many as fit about 2 s of CPU work per configuration), on the full workload
or on a stated prefix (>= 5 %) of its program ids, scaled linearly.

--workload NAME runs one workload (for profiling); --op-markers launches an
empty marker kernel before each op's own timed block, so that a rocprofv3
run can be split per op.
"""
from __future__ import annotations

import argparse
import ctypes
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
FP32_PEAK_TFLOPS = 157.3     # fp32 (vector and matrix)
CPU_PREFIX = 0.05            # minimum fraction of program ids in a sampled CPU baseline
WARM_MS = 60.0               # eager steps before a workload's step graph (clock ramp), ms of wall time
OP_WARM_MS = 10.0            # eager launches before each op's own graph (the clock is already up)


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


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class Ctx:
    """What every workload needs: the package, device, stream and options."""

    def __init__(self, args, tg, dev, stream):
        self.args, self.tg, self.dev, self.stream = args, tg, dev, stream
        self.marker = self._marker_kernel() if args.op_markers else None

    def _marker_kernel(self):
        """Marks op boundaries in a profiler's dispatch list with an empty
        launch (n = 0) of the stand-alone example kernel, whose name no op
        uses: one workgroup before each op's own block (its eager warm-up
        launches, then the warm and timed replays of its K-launch graph), two
        after a workload's last block."""
        import ctypes
        lib = self.tg._lib.lib
        mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
        self.tg.check(lib.teeny_hip_module_load(ctypes.byref(mod), self.tg._lib.EXAMPLE_MODULE_PATH.encode()))
        self.tg.check(lib.teeny_hip_module_get_function(ctypes.byref(fn), mod, b"teeny_example_axpy"))
        vals = (ctypes.c_float(0.0), ctypes.c_void_p(0), ctypes.c_void_p(0), ctypes.c_int32(0))
        argv = (ctypes.c_void_p * 4)(*(ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals))
        block = (ctypes.c_uint32 * 3)(64, 1, 1)
        keep = (mod, fn, vals, argv, block)

        def mark(blocks):
            grid = (ctypes.c_uint32 * 3)(blocks, 1, 1)
            self.tg.check(lib.teeny_hip_launch(keep[1], grid, block, 0, self.stream.handle, argv))
        return mark

    def copies(self, buf, n):
        """`buf` and n-1 device copies of it (rotating operands)."""
        out = [buf]
        for _ in range(n - 1):
            b = self.tg.Buffer(buf.dtype, buf.shape)
            self.tg.check(self.tg._lib.lib.teeny_hip_memcpy_d2d(b.ptr, buf.ptr, buf.nbytes, self.stream.handle))
            out.append(b)
        self.stream.synchronize()
        return out

    def measure(self, ops, step_ops=None, extra_steps=None):
        """ops: [(name, [launch_0, launch_1, ...])], launch_r running the op on
        rotation r.  Returns (step ms, {name: ms per launch of the op alone}).
        `step_ops` (same form, default `ops`) are what one step runs;
        `extra_steps` ({label: ops}) are timed the same way after it, into
        self.extra_step_ms."""
        tg, dev, stream = self.tg, self.dev, self.stream
        steps, warmup = self.args.steps, self.args.warmup
        step_ops = ops if step_ops is None else step_ops
        if self.marker is not None:
            log(f"[bench] ops per step: {json.dumps([n for n, _ in ops])} steps={steps}")

        def step(i):
            for _, fns in step_ops:
                fns[i % len(fns)]()

        def replay_ms(enqueue, count):
            """Captures `count` launches into one HIP graph, replays it once to
            warm up, then times one replay: ms per launch, free of host
            launch overhead (a 10-20 us kernel issued from Python otherwise
            leaves the GPU idle between launches)."""
            stream.begin_capture()
            for i in range(count):
                enqueue(i)
            g = stream.end_capture()
            g.launch(stream)
            stream.synchronize()
            t0.record(stream)
            g.launch(stream)
            t1.record(stream)
            t1.synchronize()
            g.destroy()
            return t0.elapsed_ms(t1) / count

        def warm(fn, ms):
            """Eager launches of fn(i) for at least `ms` of wall time: the
            shader clock settles under sustained load."""
            t_end = time.perf_counter() + ms / 1e3
            i = 0
            while i == 0 or time.perf_counter() < t_end:
                fn(i)
                i += 1
            dev.synchronize()

        t0, t1 = tg.Event(), tg.Event()
        for i in range(warmup):
            step(i)
        warm(step, self.args.warm_ms)
        ms = replay_ms(step, steps)
        self.extra_step_ms = {}
        for label, xops in ({} if self.args.no_extra_steps else (extra_steps or {})).items():
            def xstep(i, xops=xops):
                for _, fns in xops:
                    fns[i % len(fns)]()
            for i in range(warmup):
                xstep(i)
            warm(xstep, self.args.warm_ms)
            self.extra_step_ms[label] = replay_ms(xstep, steps)
        per = {}
        for name, fns in ops:
            if self.marker is not None:
                self.marker(1)
            warm(lambda i, fns=fns: fns[i % len(fns)](), self.args.warm_ms * OP_WARM_MS / WARM_MS)
            per[name] = replay_ms(lambda i, fns=fns: fns[i % len(fns)](), steps)
        if self.marker is not None:
            self.marker(2)
        dev.synchronize()
        return ms, per


def load_traffic(workload, op):
    """HBM bytes per launch of `op` (all its kernels) from the committed
    rocprofv3 counter summary profiles/<workload>_traffic.json, or None."""
    p = os.path.join(ROOT, "profiles", f"{workload}_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        ops = json.load(f).get("ops", {})
    entry = ops.get(op)
    return None if entry is None else entry.get("traffic_bytes_per_launch")


def roofline_bytes(workload, op, nbytes, avg_ms, per_op_bytes=None):
    ach = nbytes / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": op, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": load_traffic(workload, op),
            "algorithmic_bytes": nbytes, "avg_us": round(avg_ms * 1e3, 2)}


def roofline_flops(workload, op, flops, avg_ms, peak, nbytes=None):
    ach = flops / (avg_ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": op, "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(ach / peak, 4), "traffic": load_traffic(workload, op), "algorithmic_bytes": nbytes,
            "algorithmic_flop": flops, "avg_us": round(avg_ms * 1e3, 2)}


CPU_MIN_SECONDS = 2.0  # CPU work per configuration: about 20 s over the default run
_cpu_last = {}


def cpu_time(fn, runs=3, min_seconds=None):
    """Median wall time of at least `runs` calls, after one warm-up call, and of
    as many more as fit `min_seconds` of CPU work in total (at most 200)."""
    min_seconds = CPU_MIN_SECONDS if min_seconds is None else min_seconds
    t0 = time.perf_counter()
    fn()
    times = []
    while len(times) < runs or (time.perf_counter() - t0 < min_seconds and len(times) < 200):
        c0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - c0)
    _cpu_last.update(runs=len(times), total_seconds=round(time.perf_counter() - t0, 2))
    return float(np.median(times))


def cpu_entry(value, unit, seconds, sample, gpu_value, extra=None):
    import oracle
    d = {"value": value, "unit": unit, "cores": oracle.threads(), "kind": "port", "cpu": cpu_model(),
         "build": oracle.BUILD_FLAGS, "seconds": round(seconds, 4), "sample": sample,
         "runs": _cpu_last.get("runs"), "cpu_seconds_total": _cpu_last.get("total_seconds"),
         "speedup": round(gpu_value / value, 1) if value else None}
    if extra:
        d.update(extra)
    return d


def upload_bf16(ctx, a):
    from teenygrad_amd.dtypes import to_bf16
    return ctx.dev.upload(to_bf16(a), ctx.tg.bf16)


# ── configuration 2: norm + activation chain ───────────────────────────────

NORM_M, NORM_N = 16384, 4096


def norm_inputs():
    from teenygrad_amd import synthetic
    from teenygrad_amd.dtypes import round_bf16
    x = round_bf16(synthetic.normal(synthetic.workload_seed(1, 0), (NORM_M, NORM_N)))
    g1 = round_bf16(synthetic.normal(synthetic.workload_seed(1, 1), (NORM_N,), 1.0, 0.02))
    b1 = round_bf16(synthetic.normal(synthetic.workload_seed(1, 2), (NORM_N,), 0.0, 0.02))
    g2 = round_bf16(synthetic.normal(synthetic.workload_seed(1, 3), (NORM_N,), 1.0, 0.02))
    return x, g1, b1, g2


def bench_norm_act(ctx):
    from teenygrad_amd import kernels as K
    tg, stream = ctx.tg, ctx.stream
    x, g1, b1, g2 = norm_inputs()
    g1b, b1b, g2b = (upload_bf16(ctx, a) for a in (g1, b1, g2))
    shape = (NORM_M, NORM_N)
    R = 4  # 4 x 128 MiB of X: a launch never finds its input in the Infinity Cache
    xs = ctx.copies(upload_bf16(ctx, x), R)
    y1, gl, sl, y2, gr, sr = ([tg.Buffer(tg.bf16, shape) for _ in range(R)] for _ in range(6))
    rrms = tg.Buffer(tg.f32, (NORM_M,))
    io = 2 * NORM_M * NORM_N * 2  # read X + write Y, bf16
    bytes_of = {"layer_norm": io + 2 * NORM_N * 2, "gelu(ln)": io, "silu(ln)": io,
                "rms_norm": io + NORM_N * 2 + NORM_M * 4, "gelu(rms)": io, "silu(rms)": io}
    ops = [("layer_norm", [lambda r=r: K.layer_norm(xs[r], g1b, b1b, 1e-5, y=y1[r], stream=stream) for r in range(R)]),
           ("gelu(ln)", [lambda r=r: K.gelu(y1[r], y=gl[r], stream=stream) for r in range(R)]),
           ("silu(ln)", [lambda r=r: K.silu(y1[r], y=sl[r], stream=stream) for r in range(R)]),
           ("rms_norm", [lambda r=r: K.rms_norm(xs[r], g2b, 1e-8, y=y2[r], rrms=rrms, stream=stream)
                         for r in range(R)]),
           ("gelu(rms)", [lambda r=r: K.gelu(y2[r], y=gr[r], stream=stream) for r in range(R)]),
           ("silu(rms)", [lambda r=r: K.silu(y2[r], y=sr[r], stream=stream) for r in range(R)])]
    ms, per = ctx.measure(ops)
    step_bytes = sum(bytes_of.values())
    value = step_bytes / (ms * 1e-3) / 1e9
    # the roofline unit: LayerNorm, the op with the least headroom (two
    # dependent reductions per row); the other five are in `ops`
    roof = roofline_bytes("norm_act", "layer_norm", bytes_of["layer_norm"], per["layer_norm"])
    opsd = {k: {"us": round(v * 1e3, 2), "GB/s": round(bytes_of[k] / (v * 1e-3) / 1e9, 1),
                "frac": round(bytes_of[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "traffic": load_traffic("norm_act", k)} for k, v in per.items()}
    cpu = None
    if not ctx.args.no_cpu:
        import oracle

        def run():
            ln = oracle.layer_norm(x, g1, b1, 1e-5)
            oracle.gelu(ln)
            oracle.silu(ln)
            rm, _ = oracle.rms_norm(x, g2, 1e-8)
            oracle.gelu(rm)
            oracle.silu(rm)

        cs = cpu_time(run)
        cpu = cpu_entry(round(step_bytes / cs / 1e9, 2), "GB/s", cs,
                        "the full step (6 ops on [16384, 4096]) in fp32 on the bf16-rounded inputs; bytes "
                        "counted as bf16 like the GPU line", value)
    # the measured HBM traffic of one step (rocprofv3 FETCH_SIZE + WRITE_SIZE
    # per op, scaled by a copy of known size), when every op has a figure
    traffic = [load_traffic("norm_act", k) for k in bytes_of]
    hbm_step = sum(traffic) if all(t is not None for t in traffic) else None
    return {"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "norm_act_chain: X[16384,4096] bf16 -> LayerNorm -> GELU-tanh, SiLU; "
                                   "RMSNorm -> GELU-tanh, SiLU (fp32 stats)",
                       "M": NORM_M, "N": NORM_N, "ops_per_step": 6, "bytes_per_step": step_bytes,
                       "value_counts": "algorithmic bytes / step time; each GELU/SiLU reads the tensor the "
                                       "norm before it has just written, part of it from the 256 MB Infinity "
                                       "Cache, so the step value is not a pure HBM rate (the per-op roofline "
                                       "entries time each op on rotated, cold operands)",
                       "hbm_bytes_per_step": hbm_step,
                       "hbm_GBs": round(hbm_step / (ms * 1e-3) / 1e9, 1) if hbm_step else None},
            "roofline": roof, "cpu_baseline": cpu, "ops": opsd}


COPY_BYTES = 128 << 20


def copy_ceiling(ctx):
    """The achievable HBM rate next to the 8 TB/s datasheet peak: a plain
    device-to-device hipMemcpyAsync of 128 MiB (128 MiB read + 128 MiB
    written), over four rotating source/destination pairs so that no copy
    finds its source in the Infinity Cache, timed like every op here."""
    tg, stream = ctx.tg, ctx.stream
    R = 4
    src = [tg.Buffer(tg.i8, (COPY_BYTES,)) for _ in range(R)]
    dst = [tg.Buffer(tg.i8, (COPY_BYTES,)) for _ in range(R)]
    for b in src:
        b.zero_(stream)
    lib = tg._lib.lib
    fns = [lambda r=r: tg.check(lib.teeny_hip_memcpy_d2d(dst[r].ptr, src[r].ptr, COPY_BYTES, stream.handle))
           for r in range(R)]
    _, per = ctx.measure([("d2d_copy", fns)])
    ms = per["d2d_copy"]
    moved = 2 * COPY_BYTES
    gbs = moved / (ms * 1e-3) / 1e9
    return {"GB/s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "avg_us": round(ms * 1e3, 2),
            "bytes_per_copy": moved, "how": "hipMemcpyAsync device-to-device, 128 MiB, 4 rotating buffer pairs, "
                                           "graph-replayed; bytes = read + written"}


def bench_act_backward(ctx):
    """Activation gradients on the norm workload's shape: dy and the saved tensor in, dx out
    (relu takes the forward output, gelu/silu the forward input); 3 x 128 MiB per op."""
    from teenygrad_amd import kernels as K
    from teenygrad_amd import synthetic
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    x, _, _, _ = norm_inputs()
    dy = round_bf16(synthetic.normal(synthetic.workload_seed(1, 4), (NORM_M, NORM_N)))
    y = np.maximum(x, 0)
    R = 4
    xb, yb, dyb = (ctx.copies(upload_bf16(ctx, a), R) for a in (x, y, dy))
    shape = (NORM_M, NORM_N)
    dr, dg, ds = ([tg.Buffer(tg.bf16, shape) for _ in range(R)] for _ in range(3))
    io = 3 * NORM_M * NORM_N * 2
    bytes_of = {"relu_backward": io, "gelu_backward": io, "silu_backward": io}
    ops = [("relu_backward", [lambda r=r: K.relu_backward(dyb[r], yb[r], dx=dr[r], stream=stream) for r in range(R)]),
           ("gelu_backward", [lambda r=r: K.gelu_backward(dyb[r], xb[r], dx=dg[r], stream=stream) for r in range(R)]),
           ("silu_backward", [lambda r=r: K.silu_backward(dyb[r], xb[r], dx=ds[r], stream=stream) for r in range(R)])]
    ms, per = ctx.measure(ops)
    step_bytes = sum(bytes_of.values())
    value = step_bytes / (ms * 1e-3) / 1e9
    roof = roofline_bytes("act_backward", "gelu_backward", io, per["gelu_backward"])
    ops = {k: {"us": round(v * 1e3, 2), "GB/s": round(bytes_of[k] / (v * 1e-3) / 1e9, 1),
               "frac": round(bytes_of[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)} for k, v in per.items()}
    cpu = None
    if not ctx.args.no_cpu:
        import oracle

        def run():
            oracle.relu_backward(dy, y)
            oracle.gelu_backward(dy, x)
            oracle.silu_backward(dy, x)

        cs = cpu_time(run)
        cpu = cpu_entry(round(step_bytes / cs / 1e9, 2), "GB/s", cs,
                        "the full step (3 gradients on [16384, 4096]) in fp32 on the bf16-rounded inputs",
                        value)
    return {"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "activation gradients: dy, x|y [16384,4096] bf16 -> dx for ReLU, GELU-tanh, "
                                   "SiLU (fp32 math)", "bytes_per_step": step_bytes},
            "roofline": roof, "cpu_baseline": cpu, "ops": ops}


# ── configuration 3: attention ──────────────────────────────────────────────


def bench_attention(ctx, s, causal):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    bh, d = 256, 128
    rng = np.random.default_rng(0x7EE70002)
    host = [round_bf16(rng.standard_normal((bh, s, d), dtype=np.float32)) for _ in range(3)]
    q, k, v = (upload_bf16(ctx, a) for a in host)
    nh = math.ceil(CPU_PREFIX * bh)  # heads in the CPU baseline's prefix
    host = [np.ascontiguousarray(a[:nh]) for a in host]
    o = tg.Buffer(tg.bf16, (bh, s, d))
    lse = tg.Buffer(tg.f32, (bh, s))
    flops = 4.0 * bh * s * s * d * (0.5 if causal else 1.0)
    name = f"flash_attention_bf16_{'causal_' if causal else ''}s{s}"
    workload = f"attention_{'causal_' if causal else ''}s{s}"
    # Q/K/V/O of 512 MiB (causal S=2048) or 1 GiB exceed the Infinity Cache: no rotation
    ms, per = ctx.measure([(name, [lambda: K.flash_attention(q, k, v, None, causal, o=o, lse=lse, stream=stream)])])
    value = flops / (ms * 1e-3) / 1e12
    nbytes = 4 * bh * s * d * 2 + bh * s * 4
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        # prefix of the oracle's program grid (pid = bh * S + q_row): the first
        # ceil(5% of BH) heads, all rows; every head costs the same
        qh, kh, vh = host
        cs = cpu_time(lambda: oracle.flash_attention(qh, kh, vh, None, causal))
        frac = nh / bh
        full = cs / frac
        cpu = cpu_entry(round(flops / full / 1e12, 5), "TFLOP/s", cs,
                        f"program-id prefix: {nh} of {bh} (batch, head) pairs, all {s} query rows "
                        f"({frac:.2%} of the grid), fp32; scaled x{bh / nh:.2f}", value,
                        {"prefix_fraction": round(frac, 4), "extrapolated_seconds": round(full, 2)})
    return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": f"sdpa {'causal' if causal else 'non-causal'} bf16 B=8 H=32 S={s} D=128",
                       "flop_per_step": flops},
            "roofline": roofline_flops(workload, name, flops, per[name], BF16_PEAK_TFLOPS, nbytes),
            "cpu_baseline": cpu}


# ── configuration 4: ResNet-50 conv stack ───────────────────────────────────


def attach_workspace(ctx, sizes):
    """Gives the stream one caller-owned scratch buffer big enough for every
    op of the workload (split-K partials, space-to-depth copies); returns its
    size.  Allocated before timing, as an executor
    would."""
    need = max(list(sizes) + [0])
    if need > 0:
        ctx.stream.set_workspace(ctx.dev.buffer(ctx.tg.i8, (need,)))
    return need


def bench_resnet(ctx):
    from teenygrad_amd import kernels as K
    from teenygrad_amd import synthetic
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    B = 64
    rng = np.random.default_rng(0x7EE70003)
    layers = synthetic.resnet50_convs()
    assert len(layers) == 53
    bufs, host = [], []
    flops = 0.0
    total_bytes = 0
    for name, cin, cout, h, k, s, p, relu in layers:
        oh = (h + 2 * p - k) // s + 1
        x = round_bf16(rng.random((B, h, h, cin), dtype=np.float32))
        w = round_bf16((rng.standard_normal((cout, k, k, cin), dtype=np.float32)
                        * np.float32(np.sqrt(2.0 / (cin * k * k)))))
        b = round_bf16(rng.normal(0, 0.01, cout).astype(np.float32))
        y = tg.Buffer(tg.bf16, (B, oh, oh, cout))
        f = 2.0 * B * oh * oh * cout * cin * k * k
        nb = 2 * (B * h * h * cin + cout * k * k * cin + cout + B * oh * oh * cout)
        flops += f
        total_bytes += nb
        # two operand sets per layer, so the layer's own timed block reads HBM
        xr, wr = ctx.copies(upload_bf16(ctx, x), 2), ctx.copies(upload_bf16(ctx, w), 2)
        ys = [y, tg.Buffer(tg.bf16, (B, oh, oh, cout))]
        bufs.append((name, xr, wr, upload_bf16(ctx, b), ys, s, p, relu, f, nb))
        if not ctx.args.no_cpu:  # NCHW copies of the first images, for the oracle
            xs = np.ascontiguousarray(np.transpose(x[:math.ceil(CPU_PREFIX * B)], (0, 3, 1, 2)))
            host.append((xs, np.ascontiguousarray(np.transpose(w, (0, 3, 1, 2))), b, s, p, relu))
        del x
    ws = attach_workspace(ctx, (
        K.conv2d_workspace_size((B, h, h, cin), (cout, k, k, cin), s, p, 1, tg.bf16, "nhwc")
        for name, cin, cout, h, k, s, p, relu in layers))
    log(f"[bench] resnet50 stream workspace {ws / 2**20:.1f} MiB")

    ops = [(name, [lambda r=r, x=x, w=w, b=b, y=y, s=s, p=p, relu=relu:
                   K.conv2d(x[r], w[r], b, s, p, 1, "relu" if relu else None, "nhwc", y=y[r], stream=stream)
                   for r in range(2)])
           for name, x, w, b, y, s, p, relu, _, _ in bufs]
    # The step is the stack: each conv reads the activation the previous one
    # wrote (c1 -> c2 -> c3 -> the next block's c1; a downsample reads its
    # block's input, as c1 does; stage 1's first block reads its own buffer,
    # the stem's pooled output, which no conv writes).  Each op's own timing,
    # and the `independent_inputs` step, give every conv a separate input.
    byname = {bb[0]: bb for bb in bufs}
    chain_in, prev, block_in = {}, None, None
    for name, cin, cout, h, k, s, p, relu in layers:
        if name == "stem":
            src = None
        elif name.endswith("c1"):
            block_in = None if name == "l1b0c1" else prev
            src = block_in
        elif name.endswith("ds"):
            src = block_in
        else:
            src = prev
        chain_in[name] = src
        if not name.endswith("ds"):
            prev = name
    step_ops = []
    for name, x, w, b, y, s, p, relu, _, _ in bufs:
        src = chain_in[name]
        xin = x if src is None else byname[src][4]  # the producing conv's outputs, one per rotation
        if name == "l1b0ds":
            xin = byname["l1b0c1"][1]  # stage 1's first block: c1's own input
        step_ops.append((name, [lambda r=r, xin=xin, w=w, b=b, y=y, s=s, p=p, relu=relu:
                                K.conv2d(xin[r], w[r], b, s, p, 1, "relu" if relu else None, "nhwc", y=y[r],
                                         stream=stream)
                                for r in range(2)]))
    ms, per = ctx.measure(ops, step_ops, {"independent_inputs": ops})
    independent_ms = ctx.extra_step_ms.get("independent_inputs", float("nan"))
    value = flops / (ms * 1e-3) / 1e12
    # each layer's own floor: the longer of its MFMA time at the bf16 peak and
    # its algorithmic bytes at the HBM peak; the stack's floor is their sum
    by_layer = {}
    floor_sum = 0.0
    for bb in bufs:
        n, f, nb = bb[0], bb[8], bb[9]
        t_mfma, t_hbm = f / (BF16_PEAK_TFLOPS * 1e12) * 1e6, nb / (HBM_PEAK_GBS * 1e9) * 1e6
        floor_us = max(t_mfma, t_hbm)
        floor_sum += floor_us
        by_layer[n] = {"us": round(per[n] * 1e3, 1), "TFLOP/s": round(f / (per[n] * 1e-3) / 1e12, 1),
                       "bound": "mfma" if t_mfma >= t_hbm else "hbm", "floor_us": round(floor_us, 2),
                       "frac_of_floor": round(floor_us / (per[n] * 1e3), 4)}
    kernel_sum_us = sum(per.values()) * 1e3
    stack = {"floor_us": round(floor_sum, 1), "step_us": round(ms * 1e3, 1),
             "frac_of_floor": round(floor_sum / (ms * 1e3), 4), "alone_sum_us": round(kernel_sum_us, 1),
             "step_minus_alone_us": round(ms * 1e3 - kernel_sum_us, 1),
             "independent_inputs_step_us": None if math.isnan(independent_ms) else round(independent_ms * 1e3, 1),
             "step": "chained: each conv reads the activation the previous conv wrote (downsamples their block's "
                     "input); independent_inputs_step_us runs the same 53 convs with every conv reading its own "
                     "buffer (the step as timed before the chaining)",
             "how": "floor = sum over layers of max(FLOP / 2.5 PFLOP/s, algorithmic bytes / 8 TB/s); alone_sum = "
                    "the layers timed alone (own replay over two operand copies); a kernel trace of the step "
                    "graph shows no idle time between its kernels: the difference is the kernels running longer "
                    "inside the step (the previous layer's output written back meanwhile, weights and inputs "
                    "that are not in the Infinity Cache)"}
    dom = max(per, key=per.get)
    fdom, bdom = [(bb[8], bb[9]) for bb in bufs if bb[0] == dom][0]
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        nimg = host[0][0].shape[0]

        def run():
            for x, w, b, s, p, relu in host:
                y = oracle.conv2d_nchw(x, w, b, s, p)
                if relu:
                    oracle.relu(y)

        cs = cpu_time(run)
        frac = nimg / B
        full = cs / frac
        cpu = cpu_entry(round(flops / full / 1e12, 5), "TFLOP/s", cs,
                        f"program-id prefix: the first {nimg} of {B} images of every layer ({frac:.2%} of each "
                        f"conv grid; programs are image-major), conv+bias and ReLU in fp32 NCHW; scaled "
                        f"x{B / nimg:.0f}", value,
                        {"prefix_fraction": round(frac, 4), "extrapolated_seconds": round(full, 2)})
    ctx.stream.set_workspace(None)
    return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "resnet50 53 convs bf16 NHWC batch 64 224x224, BN folded to bias, ReLU fused",
                       "flop_per_step": flops, "bytes_per_step": total_bytes, "workspace_bytes": ws},
            "roofline": dict(roofline_flops("resnet50_convs", dom, fdom, per[dom], BF16_PEAK_TFLOPS, bdom),
                             layer_bound=by_layer[dom]["bound"], layer_floor_us=by_layer[dom]["floor_us"],
                             frac_of_layer_floor=by_layer[dom]["frac_of_floor"], stack=stack),
            "layers": by_layer, "cpu_baseline": cpu}


# ── configuration 5: W8A16 ──────────────────────────────────────────────────


def bench_w8a16(ctx):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    m = 4096
    rng = np.random.default_rng(0x7EE70005)
    problems, host, wdev = [], [], None
    for k, n in ((4096, 11008), (11008, 4096)):
        x = round_bf16(rng.standard_normal((m, k), dtype=np.float32))
        wf = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        wd = ctx.dev.upload(wf)
        q, s, _, _ = K.quantize_affine(wd, [n, k], "channel", 0)
        if wdev is None:
            wdev = (wd, n, k)
        del wd
        y = tg.Buffer(tg.bf16, (m, n))
        name = f"w8a16 {m}x{k}->{n}"
        problems.append((name, ctx.copies(upload_bf16(ctx, x), 2), ctx.copies(q, 2), s, [y, tg.Buffer(tg.bf16, (m, n))],
                         2 * m * k + n * k + 4 * n + 2 * m * n, 2.0 * m * n * k))
        if not ctx.args.no_cpu:
            host.append((x[:math.ceil(CPU_PREFIX * m)].copy(), q.to_host().reshape(n, k), s.to_host()))
    attach_workspace(ctx, (K.linear_workspace_size(m, n, k, tg.i8) for k, n in ((4096, 11008), (11008, 4096))))

    ops = [(name, [lambda r=r, x=x, q=q, s=s, y=y: K.w8a16_linear(x[r], q[r], s, y=y[r], stream=stream)
                   for r in range(2)])
           for name, x, q, s, y, _, _ in problems]
    ms, per = ctx.measure(ops)
    flops = sum(p[-1] for p in problems)
    value = flops / (ms * 1e-3) / 1e12
    ops = {p[0]: {"us": round(per[p[0]] * 1e3, 1), "TFLOP/s": round(p[-1] / (per[p[0]] * 1e-3) / 1e12, 1),
                  "traffic": load_traffic("w8a16_gemm", p[0]), "algorithmic_bytes": p[-2]} for p in problems}
    dom = max(per, key=per.get)
    fdom, bdom = [(p[-1], p[-2]) for p in problems if p[0] == dom][0]
    # the quantizer that makes these weights (quantize_affine per output
    # channel, fp32 [11008, 4096] -> int8 + scales), timed on its own
    wq, qn, qk = wdev
    wqs = ctx.copies(wq, 2)
    qq = [tg.Buffer(tg.i8, (qn, qk)) for _ in range(2)]
    qsc, qzp = tg.Buffer(tg.f32, (qn,)), tg.Buffer("i32", (qn,))
    shape = (ctypes.c_int64 * 2)(qn, qk)
    lib = tg._lib.lib
    qfns = [lambda r=r: tg.check(lib.teeny_quantize_affine(wqs[r].ptr, shape, 2, 1, 0, 1, 1, 8, qq[r].ptr, qsc.ptr,
                                                           qzp.ptr, None, stream.handle)) for r in range(2)]
    qname = f"quantize_affine [{qn},{qk}]"
    _, qper = ctx.measure([(qname, qfns)])
    qbytes = 4 * qn * qk + qn * qk + 8 * qn
    ops[qname] = {"us": round(qper[qname] * 1e3, 1), "GB/s": round(qbytes / (qper[qname] * 1e-3) / 1e9, 1),
                  "frac": round(qbytes / (qper[qname] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "algorithmic_bytes": qbytes,
                  "traffic": load_traffic("w8a16_gemm", qname),
                  "note": "offline weight preparation, not part of the step: fp32 read + int8 written + scales"}
    del wqs, qq
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        rows = math.ceil(CPU_PREFIX * m)
        deq = [(x, oracle.dequantize_affine(q, s, None, q.shape, "channel", 0)) for x, q, s in host]
        cs = cpu_time(lambda: [oracle.linear(x, w) for x, w in deq])
        frac = rows / m
        full = cs / frac
        cpu = cpu_entry(round(flops / full / 1e12, 5), "TFLOP/s", cs,
                        f"program-id prefix: output rows 0..{rows - 1} of {m} of both GEMMs ({frac:.2%}; one "
                        f"program per row), fp32 on dequantize_affine's weights; scaled x{m / rows:.2f}", value,
                        {"prefix_fraction": round(frac, 4), "extrapolated_seconds": round(full, 2)})
    ctx.stream.set_workspace(None)
    return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "w8a16 GEMMs M=4096: K=4096->N=11008 and K=11008->N=4096, int8 per-channel "
                                   "weights", "flop_per_step": flops},
            "roofline": roofline_flops("w8a16_gemm", dom, fdom, per[dom], BF16_PEAK_TFLOPS, bdom),
            "ops": ops, "cpu_baseline": cpu}


def bench_w8a16_conv(ctx):
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    B, C, H = 32, 256, 28
    rng = np.random.default_rng(0x7EE70006)
    xh = round_bf16(rng.standard_normal((B, H, H, C), dtype=np.float32))
    R = 4  # 4 x 26 MB of operands per launch set
    x = ctx.copies(upload_bf16(ctx, xh), R)
    wf = rng.normal(0, 0.02, (C, 3, 3, C)).astype(np.float32)
    q, s, _, _ = K.quantize_affine(ctx.dev.upload(wf), [C, 3, 3, C], "channel", 0)
    qs = ctx.copies(q, R)
    y = [tg.Buffer(tg.bf16, (B, H, H, C)) for _ in range(R)]
    flops = 2.0 * B * H * H * C * C * 9
    nbytes = 2 * B * H * H * C * 2 + C * 9 * C + 4 * C
    name = "w8a16_conv3x3"
    attach_workspace(ctx, [K.conv2d_workspace_size((B, H, H, C), (C, 3, 3, C), 1, 1, 1, tg.i8)])
    ms, per = ctx.measure([(name, [lambda r=r: K.w8a16_conv2d(x[r], qs[r], s, None, 1, 1, y=y[r], stream=stream)
                                   for r in range(R)])])
    value = flops / (ms * 1e-3) / 1e12
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        nimg = math.ceil(CPU_PREFIX * B)
        wd = oracle.dequantize_affine(q.to_host().reshape(-1), s.to_host(), None, [C, 3, 3, C], "channel", 0)
        xs, ws = np.transpose(xh[:nimg], (0, 3, 1, 2)), np.transpose(wd, (0, 3, 1, 2))
        cs = cpu_time(lambda: oracle.conv2d_nchw(xs, ws, None, 1, 1))
        frac = nimg / B
        full = cs / frac
        cpu = cpu_entry(round(flops / full / 1e12, 5), "TFLOP/s", cs,
                        f"program-id prefix: the first {nimg} of {B} images ({frac:.2%}), fp32 on "
                        f"dequantize_affine's weights; scaled x{B / nimg:.0f}", value,
                        {"prefix_fraction": round(frac, 4), "extrapolated_seconds": round(full, 2)})
    ctx.stream.set_workspace(None)
    return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "w8a16 conv3x3 NHWC 32x256x28x28 -> 256, p1", "flop_per_step": flops},
            "roofline": roofline_flops("w8a16_conv", name, flops, per[name], BF16_PEAK_TFLOPS, nbytes),
            "cpu_baseline": cpu}


# ── configuration 1: the reference's own fp32 conv ──────────────────────────


def bench_conv_f32(ctx):
    from teenygrad_amd import kernels as K
    tg, stream = ctx.tg, ctx.stream
    rng = np.random.default_rng(0x7EE70000)
    x = rng.standard_normal((1, 64, 56, 56), dtype=np.float32)
    w = (rng.standard_normal((64, 64, 3, 3), dtype=np.float32) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = (rng.standard_normal(64, dtype=np.float32) * 0.01).astype(np.float32)
    xb, wb, bb = ctx.dev.upload(x), ctx.dev.upload(w), ctx.dev.upload(b)
    y = tg.Buffer(tg.f32, (1, 64, 56, 56))
    flops = 2.0 * 64 * 56 * 56 * 64 * 9
    nbytes = 4 * (64 * 56 * 56 * 2 + 64 * 64 * 9 + 64)
    name = "conv2d_bias_relu_f32"

    # 1.75 MB of operands: L2-resident whatever the rotation (a latency-bound op)
    ms, per = ctx.measure([(name, [lambda: K.conv2d(xb, wb, bb, 1, 1, 1, "relu", y=y, stream=stream)])])
    value = flops / (ms * 1e-3) / 1e12
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        cs = cpu_time(lambda: oracle.relu(oracle.conv2d_nchw(x, w, b, padding=1)))
        cpu = cpu_entry(round(flops / cs / 1e12, 5), "TFLOP/s", cs,
                        "the full conv (+bias) and ReLU, the reference's two kernels", value)
    return {"value": round(value, 3), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "f32",
            "config": {"workload": "conv2d+bias+relu fp32 NCHW 1x64x56x56 -> 64, 3x3 s1 p1", "flop_per_step": flops},
            "roofline": roofline_flops("conv2d_f32", name, flops, per[name], FP32_PEAK_TFLOPS, nbytes),
            "cpu_baseline": cpu}


# ── training kernels (backward passes) ──────────────────────────────────────


def bench_norm_backward(ctx):
    """LayerNorm and RMSNorm backward on the norm workload's shape: dy, x in,
    dx out (bf16), fp32 statistics in and fp32 parameter gradients, with the
    stream workspace (per-workgroup column partials)."""
    from teenygrad_amd import kernels as K
    from teenygrad_amd import synthetic
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    x, g1, b1, g2 = norm_inputs()
    dy = round_bf16(synthetic.normal(synthetic.workload_seed(1, 4), (NORM_M, NORM_N)))
    R = 3
    xb, dyb = ctx.copies(upload_bf16(ctx, x), R), ctx.copies(upload_bf16(ctx, dy), R)
    g1b, b1b, g2b = (upload_bf16(ctx, a) for a in (g1, b1, g2))
    _, mean, rstd = K.layer_norm_train(xb[0], g1b, b1b, 1e-5, stream=stream)
    rrms = tg.Buffer(tg.f32, (NORM_M,))
    K.rms_norm(xb[0], g2b, 1e-8, rrms=rrms, stream=stream)
    shape = (NORM_M, NORM_N)
    dxl, dxr = ([tg.Buffer(tg.bf16, shape) for _ in range(R)] for _ in range(2))
    dw1, db1, dw2 = (tg.Buffer(tg.f32, (NORM_N,)).zero_(stream) for _ in range(3))
    ws = attach_workspace(ctx, [K.norm_backward_workspace_size(NORM_M, NORM_N, False)])
    io = 3 * NORM_M * NORM_N * 2  # read dy and x, write dx (bf16)
    bytes_of = {"layer_norm_backward": io + NORM_N * 2 + 8 * NORM_M + 16 * NORM_N,
                "rms_norm_backward": io + NORM_N * 2 + 4 * NORM_M + 8 * NORM_N}
    ops = [("layer_norm_backward", [lambda r=r: K.layer_norm_backward(dyb[r], xb[r], g1b, mean, rstd, dw1, db1,
                                                                      dx=dxl[r], stream=stream) for r in range(R)]),
           ("rms_norm_backward", [lambda r=r: K.rms_norm_backward(dyb[r], xb[r], g2b, rrms, dw2, dx=dxr[r],
                                                                  stream=stream) for r in range(R)])]
    ms, per = ctx.measure(ops)
    step_bytes = sum(bytes_of.values())
    value = step_bytes / (ms * 1e-3) / 1e9
    roof = roofline_bytes("norm_backward", "layer_norm_backward", bytes_of["layer_norm_backward"],
                          per["layer_norm_backward"])
    opsd = {k: {"us": round(v * 1e3, 2), "GB/s": round(bytes_of[k] / (v * 1e-3) / 1e9, 1),
                "frac": round(bytes_of[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "traffic": load_traffic("norm_backward", k)} for k, v in per.items()}
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        _, om, orr = oracle.layer_norm_train(x, g1, b1, 1e-5)
        _, orrms = oracle.rms_norm(x, g2, 1e-8)

        def run():
            oracle.layer_norm_backward(dy, x, g1, om, orr)
            oracle.rms_norm_backward(dy, x, g2, orrms)

        cs = cpu_time(run)
        cpu = cpu_entry(round(step_bytes / cs / 1e9, 2), "GB/s", cs,
                        "both backward kernels on the full [16384, 4096] in fp32 on the bf16-rounded inputs; bytes "
                        "counted as bf16 like the GPU line", value)
    ctx.stream.set_workspace(None)
    return {"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "norm backward: dy, x [16384,4096] bf16 -> dx bf16, dweight/dbias fp32 "
                                   "(LayerNorm, RMSNorm)", "bytes_per_step": step_bytes, "workspace_bytes": ws},
            "roofline": roof, "cpu_baseline": cpu, "ops": opsd}


def bench_attention_backward(ctx, s, causal):
    """dq, dk, dv of SDPA at the attention workload's shape (B=8, H=32, D=128)
    from the forward's o and lse.  Algorithmic flops: the five S^2 D products
    of the flash backward (S, dP, dV, dK, dQ), 2.5x the forward's."""
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    bh, d = 256, 128
    rng = np.random.default_rng(0x7EE70012)
    host = [round_bf16(rng.standard_normal((bh, s, d), dtype=np.float32)) for _ in range(4)]
    q, k, v, do = (upload_bf16(ctx, a) for a in host)
    o = tg.Buffer(tg.bf16, (bh, s, d))
    lse = tg.Buffer(tg.f32, (bh, s))
    K.flash_attention(q, k, v, None, causal, o=o, lse=lse, stream=stream)
    dq, dk, dv = (tg.Buffer(tg.bf16, (bh, s, d)) for _ in range(3))
    ws = attach_workspace(ctx, [K.attention_backward_workspace_size(bh, 1, s)])
    flops = 10.0 * bh * s * s * d * (0.5 if causal else 1.0)
    name = f"attention_backward_bf16_{'causal_' if causal else ''}s{s}"
    workload = f"attention_backward_{'causal_' if causal else ''}s{s}"
    ms, per = ctx.measure([(name, [lambda: K.attention_backward(q, k, v, o, do, lse, causal=causal, dq=dq, dk=dk,
                                                                dv=dv, stream=stream)])])
    value = flops / (ms * 1e-3) / 1e12
    nbytes = 8 * bh * s * d * 2 + bh * s * 4
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        nh = math.ceil(CPU_PREFIX * bh)
        qh, kh, vh, doh = (np.ascontiguousarray(a[:nh]) for a in host)
        oh, lh = oracle.flash_attention(qh, kh, vh, None, causal)
        cs = cpu_time(lambda: oracle.flash_attention_backward(qh, kh, vh, oh, doh, lh, None, causal))
        frac = nh / bh
        full = cs / frac
        cpu = cpu_entry(round(flops / full / 1e12, 5), "TFLOP/s", cs,
                        f"program-id prefix: {nh} of {bh} (batch, head) pairs, all {s} rows ({frac:.2%} of both "
                        f"grids), fp32; scaled x{bh / nh:.2f}", value,
                        {"prefix_fraction": round(frac, 4), "extrapolated_seconds": round(full, 2)})
    ctx.stream.set_workspace(None)
    return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": f"sdpa backward {'causal' if causal else 'non-causal'} bf16 B=8 H=32 S={s} "
                                   f"D=128 (dq, dk, dv)", "flop_per_step": flops, "workspace_bytes": ws},
            "roofline": roofline_flops(workload, name, flops, per[name], BF16_PEAK_TFLOPS, nbytes),
            "cpu_baseline": cpu}


CONV_BWD_LAYERS = [  # name, Cin, Cout, H, K, stride, pad: ResNet-50 layers at batch 64
    ("l2_3x3", 128, 128, 28, 3, 1, 1), ("l3_3x3_s2", 256, 256, 28, 3, 2, 1), ("l4_1x1", 512, 2048, 7, 1, 1, 0)]


def bench_conv_backward(ctx):
    """conv2d dx and dw (bf16 NHWC, batch 64) of three ResNet-50 layers, with
    the stream workspace (flipped weights, spread dy)."""
    from teenygrad_amd import kernels as K
    from teenygrad_amd.dtypes import round_bf16
    tg, stream = ctx.tg, ctx.stream
    B = 64
    rng = np.random.default_rng(0x7EE70013)
    ops, facts, host, sizes = [], {}, [], []
    for name, cin, cout, h, k, st, p in CONV_BWD_LAYERS:
        oh = (h + 2 * p - k) // st + 1
        x = round_bf16(rng.random((B, h, h, cin), dtype=np.float32))
        w = round_bf16(rng.standard_normal((cout, k, k, cin), dtype=np.float32) * np.float32(0.05))
        dy = round_bf16(rng.standard_normal((B, oh, oh, cout), dtype=np.float32))
        xb, wb, dyb = (upload_bf16(ctx, a) for a in (x, w, dy))
        dx, dw = tg.Buffer(tg.bf16, x.shape), tg.Buffer(tg.bf16, w.shape)
        f = 2.0 * B * oh * oh * cout * cin * k * k
        sizes.append(K.conv2d_backward_workspace_size(x.shape, w.shape, st, p, 1, tg.bf16, "nhwc"))
        ops.append((f"{name}.dx", [lambda dyb=dyb, wb=wb, dx=dx, xs=x.shape, st=st, p=p:
                                   K.conv2d_backward_dx(dyb, wb, xs, st, p, 1, "nhwc", dx=dx, stream=stream)]))
        ops.append((f"{name}.dw", [lambda dyb=dyb, xb=xb, dw=dw, ws_=w.shape, st=st, p=p:
                                   K.conv2d_backward_dw(dyb, xb, ws_, st, p, 1, "nhwc", dw=dw, stream=stream)]))
        nb_dx = 2 * (B * oh * oh * cout + cout * k * k * cin + B * h * h * cin)
        nb_dw = 2 * (B * oh * oh * cout + B * h * h * cin + cout * k * k * cin)
        facts[f"{name}.dx"] = (f, nb_dx)
        facts[f"{name}.dw"] = (f, nb_dw)
        if not ctx.args.no_cpu:
            nimg = math.ceil(CPU_PREFIX * B)
            host.append((np.ascontiguousarray(np.transpose(dy[:nimg], (0, 3, 1, 2))),
                         np.ascontiguousarray(np.transpose(x[:nimg], (0, 3, 1, 2))),
                         np.ascontiguousarray(np.transpose(w, (0, 3, 1, 2))), st, p))
    ws = attach_workspace(ctx, sizes)
    ms, per = ctx.measure(ops)
    flops = sum(f for f, _ in facts.values())
    value = flops / (ms * 1e-3) / 1e12
    dom = max(per, key=per.get)
    opsd = {n: {"us": round(v * 1e3, 1), "TFLOP/s": round(facts[n][0] / (v * 1e-3) / 1e12, 2)}
            for n, v in per.items()}
    cpu = None
    if not ctx.args.no_cpu:
        import oracle
        nimg = host[0][0].shape[0]

        def run():
            for dyh, xh, wh, st, p in host:
                oracle.conv2d_backward_dx(dyh, wh, xh.shape, st, p)
                oracle.conv2d_backward_dw(dyh, xh, wh.shape, st, p)

        cs = cpu_time(run)
        frac = nimg / B
        full = cs / frac
        cpu = cpu_entry(round(flops / full / 1e12, 5), "TFLOP/s", cs,
                        f"program-id prefix: the first {nimg} of {B} images of each layer ({frac:.2%}), dx and dw "
                        f"in fp32 NCHW; scaled x{B / nimg:.0f}", value,
                        {"prefix_fraction": round(frac, 4), "extrapolated_seconds": round(full, 2)})
    ctx.stream.set_workspace(None)
    return {"value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "conv2d backward dx + dw, bf16 NHWC batch 64: ResNet-50 3x3 128ch 28x28, "
                                   "3x3/2 256ch 28x28, 1x1 512->2048 7x7", "flop_per_step": flops,
                       "workspace_bytes": ws},
            "roofline": roofline_flops("conv_backward", dom, facts[dom][0], per[dom], BF16_PEAK_TFLOPS,
                                       facts[dom][1]),
            "ops": opsd, "cpu_baseline": cpu}


WORKLOADS = {
    "conv2d_f32": bench_conv_f32,
    "norm_act": bench_norm_act,
    "attention_causal_s2048": lambda c: bench_attention(c, 2048, True),
    "attention_s4096": lambda c: bench_attention(c, 4096, False),
    "resnet50_convs": bench_resnet,
    "w8a16_gemm": bench_w8a16,
    "w8a16_conv": bench_w8a16_conv,
    "act_backward": bench_act_backward,
    "norm_backward": bench_norm_backward,
    "attention_backward_causal_s2048": lambda c: bench_attention_backward(c, 2048, True),
    "conv_backward": bench_conv_backward,
}
# the default run: every configuration, in configuration order
CONFIGS = [("cfg1", "conv2d_f32"), ("cfg2", "norm_act"), ("cfg3a", "attention_causal_s2048"),
           ("cfg3b", "attention_s4096"), ("cfg4", "resnet50_convs"), ("cfg5a", "w8a16_gemm"),
           ("cfg5b", "w8a16_conv"),
           # the training kernels at the same shapes (not a headline configuration)
           ("train_act", "act_backward"), ("train_norm", "norm_backward"),
           ("train_attention", "attention_backward_causal_s2048"), ("train_conv", "conv_backward")]


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warm-ms", type=float, default=WARM_MS,
                    help="wall time of eager warm-up steps before each step graph (ops get "
                         f"{OP_WARM_MS / WARM_MS:.3g}x of it); 0: one step, as the counter runs use")
    ap.add_argument("--workload", default="all", choices=["all"] + sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline legs")
    ap.add_argument("--op-markers", action="store_true",
                    help="an empty marker launch after every op (splits a rocprofv3 run per op)")
    ap.add_argument("--no-extra-steps", action="store_true",
                    help="skip the second step timing of a workload (the ResNet stack with independent "
                         "inputs), as the profiler runs do: one step graph per workload under the tracer")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="first run one device-to-device copy of BYTES (a reference kernel of known "
                         "traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} requested); "
              f"run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import teenygrad_amd as tg

    dev = tg.open(int(os.environ.get("LOCAL_RANK", "0")))
    stream = tg.Stream.create()
    ctx = Ctx(args, tg, dev, stream)
    log(f"[bench] {args.workload} steps={args.steps} warmup={args.warmup} on {dev.info()['arch']}")
    if not args.no_cpu:
        import oracle
        flags = oracle.use_native_build()
        oracle.set_threads(cpu_threads())
        log(f"[bench] cpu baseline: oracle {flags}, {oracle.threads()} threads, {cpu_model()}")
    if args.copy_calibration:
        src, dst = tg.Buffer(tg.i8, (args.copy_calibration,)), tg.Buffer(tg.i8, (args.copy_calibration,))
        src.zero_(stream)
        tg.check(tg._lib.lib.teeny_hip_memcpy_d2d(dst.ptr, src.ptr, args.copy_calibration, stream.handle))
        stream.synchronize()
        del src, dst
    t_start = time.perf_counter()
    if args.workload == "all":
        configs = {}
        for key, name in CONFIGS:
            c0 = time.perf_counter()
            r = WORKLOADS[name](ctx)
            r["workload_name"] = name
            configs[key] = r
            log(f"[bench] {key} {name}: {r['value']} {r['unit']} (frac {r['roofline']['frac']}) "
                f"in {time.perf_counter() - c0:.1f} s")
        res = dict(configs["cfg2"])
        res["configs"] = configs
        res["copy_ceiling"] = copy_ceiling(ctx)
        log(f"[bench] copy ceiling: {res['copy_ceiling']['GB/s']} GB/s")
    else:
        res = WORKLOADS[args.workload](ctx)
    line = {"metric": METRIC, "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": res.pop("dtype"),
            "data": "synthetic (seeded N(0,1) / U(0,1) inputs, random-init params)"}
    line.update(res)
    line["wall_s"] = round(time.perf_counter() - t_start, 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
