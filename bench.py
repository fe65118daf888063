"""Benchmark of the MI355X tensor hot path (liboxide_hip.so) -- one JSON line on stdout.

Headline workload: BatchNorm2d training forward + backward, fp32
NCHW [64, 128, 56, 56].  One step = forward reduce (partial channel sums of x), forward apply (finalize
mean / inverse std / running update + y), backward reduce (partial sums of g and g * x_hat,
formed once) and backward input (finalize dweight / dbias + dx), launched through the C ABI on
one stream.
Algorithmic bytes per step: forward 3T + backward 5T, T = 102 760 448 B (x read by the
statistics; x read + y written by apply; g, x read by the affine reduction; g, x read + dx
written by the input backward).  ``value`` = 8T / step time in GB/s, inputs resident in HBM.

MALL (256 MB last-level cache) is defeated for the headline: steps rotate over 4 independent
input/output sets (1.6 GB), so each step's x and g were last touched three steps (1.2 GB of
traffic) earlier.  The K timed steps are launched directly on one stream with an event between
consecutive steps: ``ms_per_step`` is the median of the K per-step samples, p10 / p90 and the
mean over all K steps are reported beside it.  The same K steps as K launches of one-step
hipGraphs, and as K / 4 launches of a four-step hipGraph, are reported beside the headline
(each hipGraphLaunch adds a fixed ~5 us on the device).  Per-kernel durations for the
roofline come from HIP events that each dispatch records at its own start and end
(oxh_time_next_launch, i.e. hipExtLaunchKernelGGL) in a separate eager pass before the
headline's.  The secondary workloads warm up for at least 30 ms of device time before their
timed repetitions.

The other configs (elementwise chain + JIT-plan replay, cross entropy, AdamW) are measured
after the headline and reported under "extra" in the same line.  ``cpu_baseline`` times the
oracle (a single-threaded C restatement of the reference CPU path) on one BN step.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (REPO / "oxide-beta_amd", REPO / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

PEAK_HBM_GBS = 8000.0
EXTRAS = ("elementwise", "cross_entropy", "adamw", "mnist_step")
T_BN = 64 * 128 * 56 * 56 * 4


def _events(n):
    import torch

    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _stats(samples):
    """mean / median / p10 / p90 of a list of per-repetition times."""
    q = sorted(samples)
    pct = lambda f: q[min(len(q) - 1, int(f * len(q)))]  # noqa: E731
    return {"mean": sum(q) / len(q), "median": pct(0.5), "p10": pct(0.1), "p90": pct(0.9),
            "reps": len(q)}


def _timed_reps(stream, fn, reps: int, warmup: int = 3, warm_ms: float = 30.0):
    """Runs ``fn`` ``reps`` times back to back on ``stream`` with an event between
    consecutive repetitions (rep i = event i -> event i + 1, no gaps left out); returns the
    per-repetition statistics in microseconds.  Warm-up: at least ``warmup`` untimed
    repetitions and at least ``warm_ms`` of device time (the GPU reaches its steady clocks
    some milliseconds into a streaming workload: the first ~5 ms of 0.4 ms cross-entropy
    launches run up to 10 % slower)."""
    done, spent = 0, 0.0
    while done < warmup or (spent < warm_ms and done < 1000):
        e0, e1 = _events(2)
        e0.record(stream)
        for _ in range(max(1, warmup)):
            fn()
        e1.record(stream)
        e1.synchronize()
        spent += e0.elapsed_time(e1)
        done += max(1, warmup)
    evs = _events(reps + 1)
    evs[0].record(stream)
    for i in range(reps):
        fn()
        evs[i + 1].record(stream)
    evs[-1].synchronize()
    st = _stats([evs[i].elapsed_time(evs[i + 1]) * 1e3 for i in range(reps)])
    return {k: (round(v, 2) if k != "reps" else v) for k, v in st.items()}


def _read_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if one exists."""
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        return data.get(kernel, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def bench_batch_norm(m, steps: int, warmup: int, sets: int = 4):
    import numpy as np
    import torch

    dev = torch.device("cuda:0")
    n, c, h, w = 64, 128, 56, 56
    r = np.random.default_rng(0x6F78696400000002)
    gamma = torch.from_numpy(r.uniform(0.5, 1.5, c).astype(np.float32)).to(dev)
    beta = torch.from_numpy(r.uniform(-0.1, 0.1, c).astype(np.float32)).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x6F78696400000002)
    xs = [torch.randn((n, c, h, w), generator=gen, device=dev) for _ in range(sets)]
    gs = [torch.randn((n, c, h, w), generator=gen, device=dev) for _ in range(sets)]
    ys = [torch.empty_like(xs[0]) for _ in range(sets)]
    dxs = [torch.empty_like(xs[0]) for _ in range(sets)]
    rm, rv = torch.zeros(c, device=dev), torch.ones(c, device=dev)
    mean, inv = torch.empty(c, device=dev), torch.empty(c, device=dev)
    dw, db = torch.empty(c, device=dev), torch.empty(c, device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()

    names = ["bn_forward_reduce", "bn_forward_apply", "bn_backward_reduce", "bn_backward_input"]
    bytes_per = {"bn_forward_reduce": T_BN, "bn_forward_apply": 2 * T_BN,
                 "bn_backward_reduce": 2 * T_BN, "bn_backward_input": 3 * T_BN}

    def step(i, timers=None):
        k = i % sets
        x, g, y, dx = xs[k], gs[k], ys[k], dxs[k]
        if timers:
            timers[0].arm()
        m.batch_norm_forward_reduce(x, stream=s)
        if timers:
            timers[1].arm()
        m.batch_norm_forward_apply(x, gamma, beta, rm, rv, mean, inv, y, 0.1, 1e-5, stream=s)
        if timers:
            timers[2].arm()
        m.batch_norm_backward_reduce(g, x, mean, inv, stream=s)
        if timers:
            timers[3].arm()
        m.batch_norm_backward_input(g, x, gamma, mean, inv, dx, dw, db, stream=s)

    import oxide_hip as ox

    for i in range(warmup):
        step(i)
    s.synchronize()
    # per-kernel durations: each dispatch records its own start / stop events
    timers = [[ox.KernelTimer() for _ in names] for _ in range(steps)]
    start, stop = _events(2)
    start.record(s)
    for i in range(steps):
        step(warmup + i, timers[i])
    stop.record(s)
    s.synchronize()
    total_ms = start.elapsed_time(stop)
    per_kernel = {nm: [] for nm in names}
    for tm in timers:
        for j, nm in enumerate(names):
            per_kernel[nm].append(tm[j].elapsed_ms())
    kernels = {}
    for nm in names:
        avg_ms = sum(per_kernel[nm]) / len(per_kernel[nm])
        q = sorted(per_kernel[nm])
        pct = lambda f: round(q[min(len(q) - 1, int(f * len(q)))] * 1e3, 2)  # noqa: E731
        kernels[nm] = {"avg_us": round(avg_ms * 1e3, 2),
                       "p10_us": pct(0.1), "median_us": pct(0.5), "p90_us": pct(0.9),
                       "alg_bytes": bytes_per[nm],
                       "gbs": round(bytes_per[nm] / (avg_ms * 1e-3) / 1e9, 1)}
    event_ms_per_step = total_ms / steps
    # eager launches without the per-kernel events
    e_start, e_stop = _events(2)
    e_start.record(s)
    for i in range(steps):
        step(i)
    e_stop.record(s)
    s.synchronize()
    eager_ms = e_start.elapsed_time(e_stop) / steps
    # headline: the K timed steps launched directly on one stream, rotating over the input
    # sets, an event between consecutive steps: K per-step samples; ms_per_step is their
    # median (an event costs the stream ~2 us)
    for i in range(warmup):
        step(i)
    evs = _events(steps + 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record(s)
    for i in range(steps):
        step(i)
        evs[i + 1].record(s)
    s.synchronize()
    wall_headline = time.perf_counter() - t0
    per_step = _stats([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)])
    mean_ms = evs[0].elapsed_time(evs[-1]) / steps
    # beside it, the same K steps as K hipGraph launches, one step per graph (four one-step
    # graphs, one per input set, launched round-robin), an event between launches: each
    # hipGraphLaunch adds a fixed ~5 us on the device
    graphs = [ox.HipGraphExec.capture(s, lambda k=k: step(k)) for k in range(sets)]
    for i in range(warmup):
        graphs[i % sets].launch(s)
    s.synchronize()
    evs = _events(steps + 1)
    evs[0].record(s)
    for i in range(steps):
        graphs[i % sets].launch(s)
        evs[i + 1].record(s)
    s.synchronize()
    graph_step = _stats([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)])
    graph_step["launches"] = steps
    graph_step["steps_per_graph"] = 1
    del graphs
    # and one hipGraph of a whole rotation (four steps) per launch, K / 4 launches, which
    # spreads one launch's cost over four steps
    group = sets if steps % sets == 0 else 1
    g4 = ox.HipGraphExec.capture(s, lambda: [step(k) for k in range(group)])
    for _ in range(max(1, -(-warmup // group))):
        g4.launch(s)
    s.synchronize()
    evs = _events(steps // group + 1)
    evs[0].record(s)
    for i in range(steps // group):
        g4.launch(s)
        evs[i + 1].record(s)
    s.synchronize()
    rotation = _stats([evs[i].elapsed_time(evs[i + 1]) / group for i in range(steps // group)])
    rotation["launches"] = steps // group
    rotation["steps_per_graph"] = group
    del g4
    # hot-cache reference: the same step repeated on one input set (x, g fit in the MALL)
    hot_start, hot_stop = _events(2)
    hot_start.record(s)
    for i in range(steps):
        step(0)
    hot_stop.record(s)
    s.synchronize()
    hot_ms = hot_start.elapsed_time(hot_stop) / steps
    return dict(ms_per_step=per_step["median"], per_step=per_step, mean_ms=mean_ms,
                graph_step=graph_step, rotation=rotation, eager_ms_per_step=eager_ms,
                event_ms_per_step=event_ms_per_step, wall_ms_per_step=wall_headline * 1e3 / steps,
                kernels=kernels, hot_ms_per_step=hot_ms, sets=sets, steps=steps)


def bench_elementwise(m, reps: int = 20, plan_reps: int = 100):
    import numpy as np
    import torch

    import jit
    import oxide_hip as ox

    dev = torch.device("cuda:0")
    n = 4096 * 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x6F78696400000001)
    sets = 2
    abc = [[torch.rand(n, generator=gen, device=dev) * 2 - 1 for _ in range(3)]
           for _ in range(sets)]
    y = [torch.empty(n, device=dev) for _ in range(sets)]
    d = [[torch.empty(n, device=dev) for _ in range(3)] for _ in range(sets)]
    s = torch.cuda.Stream()
    torch.cuda.synchronize()

    def timed(fn):
        counter = iter(range(1 << 30))
        return _timed_reps(s, lambda: fn(next(counter)), reps)

    fwd_st = timed(lambda i: m.elementwise_chain_forward(*abc[i % sets], y[i % sets], stream=s))
    bwd_st = timed(lambda i: m.elementwise_chain_backward(*abc[i % sets], None, *d[i % sets],
                                                          stream=s))
    fwd, bwd = fwd_st["median"], bwd_st["median"]
    # the reference's JIT plan: add -> mul -> relu over three workspaces; compile fuses the
    # dependent run into one kernel (a, b, c read, y written) captured into a graph
    rr = np.random.default_rng(0x6F78696400000001)
    host = [rr.uniform(-1, 1, (4096, 4096)).astype(np.float32) for _ in range(3)]
    module = jit.trace(host, lambda i: ((i[0] + i[1]) * i[2]).relu())
    module.run(host)
    plan = module.plan_for(((4096, 4096),) * 3)
    pstream = plan.stream()
    ext = torch.cuda.ExternalStream(pstream)
    # µs per plan replay: back-to-back hipGraph launches (cuda_graph.rs:157-164), an event
    # between consecutive replays; beside it the same kernel issued without the graph
    replay = _timed_reps(ext, plan.replay, plan_reps)
    direct = _timed_reps(ext, plan.launch, plan_reps)
    # host time of one replay call (Python -> ctypes -> hipGraphLaunch), no wait in between:
    # the queue stays ahead of the device when this is below the kernel time
    host_us = []
    for _ in range(plan_reps):
        t0 = time.perf_counter()
        plan.replay()
        host_us.append((time.perf_counter() - t0) * 1e6)
    ox.check(ox.lib().oxh_stream_synchronize(pstream))
    ox.check(ox.lib().oxh_stream_synchronize(pstream))
    t0 = time.perf_counter()
    for _ in range(3):
        module.run(host)
    run_us = (time.perf_counter() - t0) / 3 * 1e6
    plan.close()
    return {
        "config": "relu((a+b)*c) fp32 3x[4096,4096]",
        "fused_fwd_us": fwd, "fused_fwd_gbs": round(4 * n * 4 / fwd / 1e3, 1),
        "fused_fwd": fwd_st,
        "fused_bwd_us": bwd, "fused_bwd_gbs": round(6 * n * 4 / bwd / 1e3, 1),
        "fused_bwd": bwd_st,
        "plan_replay_us": replay["median"],
        "plan_replay": replay,
        "plan_replay_gbs": round(4 * n * 4 / replay["median"] / 1e3, 1),
        "plan_replay_host_call_us": round(sorted(host_us)[len(host_us) // 2], 2),
        "plan_direct_launch_us": direct["median"],
        "plan_direct_launch": direct,
        "plan_run_with_copies_us": round(run_us, 1),
    }


def bench_cross_entropy(m, reps: int = 50):
    import torch

    dev = torch.device("cuda:0")
    b, k = 8192, 32768
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x6F78696400000003)
    logits = torch.randn((b, k), generator=gen, device=dev) * 2.0
    targets = torch.randint(0, k, (b,), generator=gen, device=dev).float()
    grad = torch.empty_like(logits)
    loss = torch.empty(1, device=dev)
    outer = torch.ones(1, device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()

    fused_st = _timed_reps(s, lambda: m.cross_entropy_forward_backward(
        b, k, logits, targets, outer, loss, grad, stream=s), reps, warmup=10)
    fwd_st = _timed_reps(s, lambda: m.cross_entropy_forward(b, k, logits, targets, loss,
                                                            stream=s), reps, warmup=10)
    fused, fwd = fused_st["median"], fwd_st["median"]
    L = b * k * 4
    return {"config": "CE fp32 [8192,32768]", "fused_fwd_bwd_us": fused,
            "fused_fwd_bwd_gbs": round(2 * L / fused / 1e3, 1), "fused_fwd_bwd": fused_st,
            "fwd_us": fwd, "fwd_gbs": round(L / fwd / 1e3, 1), "fwd": fwd_st}


def bench_adamw(m, reps: int = 50):
    import torch

    import oxide_hip as ox

    dev = torch.device("cuda:0")
    n = 64 << 20
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x6F78696400000004)
    p = torch.randn(n, generator=gen, device=dev) * 0.02
    g = torch.randn(n, generator=gen, device=dev) * 1e-3
    gp = torch.randn(n, generator=gen, device=dev) * 1e-3
    mom = gp * 0.1
    vel = gp * gp * 0.001
    c1, c2 = ox.adamw_corrections(0.9, 0.999, 10)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()

    def fn():
        m.adamw(1e-3, 0.01, 0.9, 0.999, c1, c2, 1e-8, p, g, mom, vel, p, mom, vel, stream=s)

    st = _timed_reps(s, fn, reps, warmup=10)
    us = st["median"]
    return {"config": "AdamW fp32 64Mi elements t=10", "us": us, "reps": st,
            "gbs": round(7 * n * 4 / us / 1e3, 1),
            "frac_of_peak": round(7 * n * 4 / us / 1e3 / PEAK_HBM_GBS, 3)}


def bench_mnist_step(steps: int = 20, batch: int = 128):
    """Config 5: the MobileNetV4-Conv-S MNIST training step (forward, cross entropy,
    backward, AdamW) as one hipGraph replay; synthetic batch (pixels k / 255, labels 0-9)."""
    import numpy as np
    import torch

    import training as T

    step = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), batch)
    r = np.random.default_rng(0x6F78696400000005)
    step.set_batch((r.integers(0, 256, (batch, 1, 28, 28)) / 255.0).astype(np.float32),
                   r.integers(0, 10, batch).astype(np.float32))

    def timed(fn, reps):
        e0, e1 = _events(2)
        e0.record(step.stream)
        for _ in range(reps):
            fn()
        e1.record(step.stream)
        step.synchronize()
        return e0.elapsed_time(e1) / reps

    step.run_eager()
    eager_ms = timed(step.run_eager, 3)
    # per launch group: events on the step's stream around each group (eager; the events add
    # a small gap between groups, so shares are of the summed group times)
    pairs = [_events(2) for _ in step.ops]
    for op, (e0, e1) in zip(step.ops, pairs):
        e0.record(step.stream)
        op.launch()
        e1.record(step.stream)
    step.synchronize()
    kinds = {}
    for op, (e0, e1) in zip(step.ops, pairs):
        category, nbytes = T.op_bytes(op)
        k = kinds.setdefault(category, {"groups": 0, "us": 0.0, "alg_bytes": 0})
        k["groups"] += 1
        k["us"] += e0.elapsed_time(e1) * 1e3
        k["alg_bytes"] += nbytes
    total_us = sum(k["us"] for k in kinds.values())
    for k in kinds.values():
        k["share"] = round(k["us"] / total_us, 4)
        k["gbs"] = round(k["alg_bytes"] / (k["us"] * 1e-6) / 1e9, 1) if k["alg_bytes"] else None
        k["us"] = round(k["us"], 1)
    step.capture()
    replay_st = _timed_reps(step.stream, step.replay, max(steps, 50))
    graph_ms = replay_st["median"] / 1e3
    loss = step.loss_value()
    return {"config": f"MobileNetV4-Conv-S MNIST train step, batch {batch}, fp32",
            "graph_ms_per_step": round(graph_ms, 4), "graph_replay_us": replay_st,
            "eager_ms_per_step": round(eager_ms, 3),
            "images_per_s": round(batch / (graph_ms * 1e-3), 1),
            "launch_groups_per_step": len(step.ops), "steps_timed": replay_st["reps"],
            "parameters": step.model.parameter_count(), "loss_after": round(loss, 5),
            "per_kind": kinds}


def copy_calibration():
    """Three 1 GiB device-to-device copies (hipMemcpyAsync's blit kernel): a plain copy of
    known traffic (1 GiB read + 1 GiB written per launch) for scaling HBM counters."""
    import torch

    import oxide_hip as ox

    src = torch.zeros(1 << 28, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        ox.check(ox.lib().oxh_memcpy_d2d_async(dst.data_ptr(), src.data_ptr(), 1 << 30, 0))
    torch.cuda.synchronize()


def copy_ceiling(reps: int = 10):
    """The streaming ceilings the kernels above are read against: 1 GiB device-to-device
    copies (1 GiB read + 1 GiB written each), timed with events over `reps` back-to-back
    copies -- torch's vectorized elementwise copy kernel and hipMemcpyAsync's blit kernel."""
    import torch

    import oxide_hip as ox

    src = torch.zeros(1 << 28, device="cuda")
    dst = torch.empty_like(src)
    s = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(2):
            fn()
        e0, e1 = _events(2)
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        e1.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        return {"us": round(us, 1), "gbs": round(2 * (1 << 30) / (us * 1e-6) / 1e9, 1)}

    out = {"what": "1 GiB device-to-device copy (2 GiB traffic)",
           "torch_copy": timed(lambda: dst.copy_(src)),
           "hip_memcpy": timed(lambda: ox.check(ox.lib().oxh_memcpy_d2d_async(
               dst.data_ptr(), src.data_ptr(), 1 << 30, s.cuda_stream)))}
    del src, dst
    torch.cuda.empty_cache()
    return out


class _OneCore:
    """Pins the process to one core for the duration (the reference's CPU path is
    single-threaded)."""

    def __enter__(self):
        self.affinity = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else None
        self.core = min(self.affinity) if self.affinity else None
        if self.core is not None:
            os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        if self.core is not None:
            os.sched_setaffinity(0, self.affinity)


def _cpu_time(fn, reps: int = 3):
    fn()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_other_configs():
    """The oracle (one core) on configs 1, 3 and 4, timed beside the GPU figures: 1 warm-up and
    the median of 3 repetitions each, GB/s over the same algorithmic bytes as the GPU lines."""
    import numpy as np

    import oracle

    out = {}
    with _OneCore() as pin:
        r = np.random.default_rng(0x6F78696400000001)
        n = 4096 * 4096
        a, b, c = (r.uniform(-1, 1, n).astype(np.float32) for _ in range(3))
        fwd = _cpu_time(lambda: oracle.relu(oracle.mul(oracle.add(a, b), c)))
        bwd = _cpu_time(lambda: oracle.chain_backward_ones(a, b, c))
        out["elementwise"] = {
            "sample": "relu((a+b)*c) on 3x[4096,4096]: forward as the CPU plan's three passes, "
                      "backward of sum()",
            "fwd_ms": round(fwd * 1e3, 1), "fwd_gbs": round(8 * n * 4 / fwd / 1e9, 2),
            "bwd_ms": round(bwd * 1e3, 1), "bwd_gbs": round(6 * n * 4 / bwd / 1e9, 2)}
        rows, classes = 8192, 32768
        r = np.random.default_rng(0x6F78696400000003)
        logits = r.standard_normal((rows, classes), dtype=np.float32) * np.float32(2.0)
        targets = r.integers(0, classes, rows).astype(np.float32)
        t0 = time.perf_counter()
        oracle.ce_forward(logits, targets)
        oracle.ce_backward(logits, targets, 1.0)
        ce = time.perf_counter() - t0
        del logits
        out["cross_entropy"] = {
            "sample": "config 3 in full (8192 rows x 32768 classes): loss + gradient, one run",
            "ms": round(ce * 1e3, 1), "gbs": round(2 * rows * classes * 4 / ce / 1e9, 2)}
        n = 64 << 20
        r = np.random.default_rng(0x6F78696400000004)
        p = (r.standard_normal(n, dtype=np.float32) * 0.02)
        g = (r.standard_normal(n, dtype=np.float32) * 1e-3)
        m = (r.standard_normal(n, dtype=np.float32) * 1e-4)
        v = np.abs(r.standard_normal(n, dtype=np.float32)) * 1e-9
        aw = _cpu_time(lambda: oracle.adamw_update(p, g, m, v, 10))
        out["adamw"] = {"sample": "config 4: 64Mi elements, t=10", "ms": round(aw * 1e3, 1),
                        "gbs": round(7 * n * 4 / aw / 1e9, 2)}
        out["cores"] = 1
        out["pinned_core"] = pin.core
    return out


def cpu_baseline(budget_s: float = 12.0):
    """The oracle (single-threaded C restatement of the reference CPU path) on one full BN
    step at config 2: forward (statistics, running update, apply) + backward."""
    import numpy as np

    import oracle

    r = np.random.default_rng(0x6F78696400000002)
    shape = (64, 128, 56, 56)
    x = r.standard_normal(shape, dtype=np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    gamma = r.uniform(0.5, 1.5, 128).astype(np.float32)
    beta = r.uniform(-0.1, 0.1, 128).astype(np.float32)
    rm, rv = np.zeros(128, np.float32), np.ones(128, np.float32)
    # one core, as the reference's CPU path runs (no threading): pinned for the timing
    affinity = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else None
    core = min(affinity) if affinity else None
    if core is not None:
        os.sched_setaffinity(0, {core})
    try:
        y, mean, inv, rm, rv = oracle.bn_forward(x, gamma, beta, rm, rv)  # warm-up step
        oracle.bn_backward(g, x, gamma, mean, inv, True)
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            y, mean, inv, rm, rv = oracle.bn_forward(x, gamma, beta, rm, rv)
            oracle.bn_backward(g, x, gamma, mean, inv, True)
            times.append(time.perf_counter() - t0)
    finally:
        if core is not None:
            os.sched_setaffinity(0, affinity)
    best = sorted(times)[len(times) // 2]
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next(line.split(":", 1)[1].strip() for line in f
                             if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": round(8 * T_BN / best / 1e9, 2), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{len(times)} full config-2 BN fwd+bwd steps after one warm-up (median "
                      f"{best * 1e3:.0f} ms per step) of oracle/oxide_oracle.c, single thread "
                      f"pinned to core {core}",
            "host": {"cpu": cpu_model, "nproc": os.cpu_count(),
                     "affinity_cores": len(affinity) if affinity else None}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true", help="headline BN config only")
    ap.add_argument("--extras", default=",".join(EXTRAS),
                    help="comma-separated secondary workloads measured after the headline "
                         f"(default: all of {','.join(EXTRAS)})")
    ap.add_argument("--only", choices=EXTRAS,
                    help="run one secondary workload alone and print its result (for "
                         "profiling that workload's kernels)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device-to-device copy (3 launches) whose known "
                         "traffic calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the hot path has no multi-GPU "
              "component); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import oxide_hip as ox

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    m = ox.load_kernels(0)
    if args.only:
        runners = {"elementwise": lambda: bench_elementwise(m),
                   "cross_entropy": lambda: bench_cross_entropy(m),
                   "adamw": lambda: bench_adamw(m),
                   "mnist_step": lambda: bench_mnist_step(args.steps)}
        print(json.dumps({"workload": args.only, **runners[args.only]()}), flush=True)
        return
    bn = bench_batch_norm(m, args.steps, args.warmup)
    dominant = max(bn["kernels"], key=lambda k: bn["kernels"][k]["avg_us"])
    dk = bn["kernels"][dominant]
    achieved = dk["alg_bytes"] / (dk["avg_us"] * 1e-6) / 1e9
    value = 8 * T_BN / (bn["ms_per_step"] * 1e-3) / 1e9
    extra = {"bn_kernels": bn["kernels"],
             "bn_hot_cache_gbs": round(8 * T_BN / (bn["hot_ms_per_step"] * 1e-3) / 1e9, 1),
             "bn_frac_of_peak": round(value / PEAK_HBM_GBS, 3),
             "bn_eager_ms_per_step": round(bn["eager_ms_per_step"], 4),
             "bn_eager_gbs": round(8 * T_BN / (bn["eager_ms_per_step"] * 1e-3) / 1e9, 1),
             "bn_events_ms_per_step": round(bn["event_ms_per_step"], 4),
             "bn_step_ms": {"median": round(bn["per_step"]["median"], 4),
                            "p10": round(bn["per_step"]["p10"], 4),
                            "p90": round(bn["per_step"]["p90"], 4),
                            "mean": round(bn["mean_ms"], 4), "samples": bn["per_step"]["reps"],
                            "what": "per step: the four kernels launched directly, an event "
                                    "between consecutive steps (one sample per timed step); "
                                    "mean = all K steps between the first and last event"},
             "bn_gbs_p10_p90": [round(8 * T_BN / (bn["per_step"]["p90"] * 1e-3) / 1e9, 1),
                                round(8 * T_BN / (bn["per_step"]["p10"] * 1e-3) / 1e9, 1)],
             "bn_graph_step_ms": {k: round(v, 4) if isinstance(v, float) else v
                                  for k, v in bn["graph_step"].items()},
             "bn_rotation_graph_step_ms": {k: round(v, 4) if isinstance(v, float) else v
                                           for k, v in bn["rotation"].items()},
             "copy_ceiling": copy_ceiling()}
    chosen = [] if args.no_extra else [e for e in args.extras.split(",") if e]
    for name in chosen:
        if name not in EXTRAS:
            print(f"bench.py: unknown workload {name!r}", file=sys.stderr)
            sys.exit(2)
    runners = {"elementwise": lambda: bench_elementwise(m),
               "cross_entropy": lambda: bench_cross_entropy(m),
               "adamw": lambda: bench_adamw(m), "mnist_step": lambda: bench_mnist_step()}
    for name in chosen:
        extra[name] = runners[name]()
    out = {
        "metric": "BatchNorm2d train fwd+bwd achieved HBM bandwidth (algorithmic bytes)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(bn["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (x, g ~ N(0,1) seeded; gamma ~ U(0.5,1.5), beta ~ U(-0.1,0.1))",
        "config": {"workload": "BatchNorm2d train fwd+bwd NCHW [64,128,56,56] fp32, momentum "
                               "0.1, eps 1e-5, 4 rotating input sets (MALL-flushed), direct "
                               "launches, an event per step",
                   "algorithmic_bytes_per_step": 8 * T_BN},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 3),
                     "traffic": _read_traffic(dominant),
                     "traffic_source": "profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE, "
                                       "WRITE_SIZE per dispatch of this kernel, scaled by a "
                                       "1 GiB copy; L2-to-fabric bytes, Infinity Cache (MALL) "
                                       "hits included, not measured in this run",
                     "achieved_from": "algorithmic bytes / average dispatch duration (HIP "
                                      "events recorded by each dispatch, eager pass)"},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(),
        "extra": extra,
    }
    if not args.no_cpu and not args.no_extra:
        extra["cpu_other_configs"] = cpu_other_configs()
    if args.copy_calibration:
        copy_calibration()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
