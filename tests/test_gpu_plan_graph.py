"""JIT plans and graph replay on the GPU: the reference's trace / compile KATs (jit.rs:721-761),
config 1's relu((a+b)*c) plan at [4096, 4096] against the oracle, and captured batch-norm /
cross-entropy / AdamW sequences replayed several times with eager work in between, every replay
checked against the eager result."""

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
from helpers import assert_bitexact, host, to_dev

pytestmark = pytest.mark.gpu


def test_trace_caches_and_reuses_a_graph():
    """jit.rs:721-736: relu(x + bias) with bias [1, 1] on [-2, 3] -> [0, 4]; one plan."""
    module = ox.trace(lambda x: (x + ox.constant([1.0, 1.0])).relu())
    assert module.run(np.array([-2.0, 3.0], np.float32)).tolist() == [0.0, 4.0]
    assert module.cached_specializations() == 1
    assert module.run(np.array([5.0, -7.0], np.float32)).tolist() == [6.0, 0.0]
    assert module.cached_specializations() == 1


def test_compile_specializes_per_shape():
    module = ox.compile(lambda a, b: (a * b).relu())
    assert module.run(np.array([1, -1], np.float32), np.array([2, 2], np.float32)).tolist() \
        == [2.0, 0.0]
    assert module.run(np.ones((2, 3), np.float32), np.ones((2, 3), np.float32)).shape == (2, 3)
    assert module.cached_specializations() == 2
    with pytest.raises(ox.OxideError) as err:
        module.plan_for(((2,), (2,))).run([np.ones(2, np.float32)])  # one input missing
    assert err.value.kind == "Trace"


def test_config1_plan_matches_oracle():
    """Config 1 via compile: relu((a+b)*c), three [4096, 4096] inputs, values U(-1, 1)."""
    r = np.random.default_rng(0x6F78696400000001)
    a, b, c = (r.uniform(-1, 1, (4096, 4096)).astype(np.float32) for _ in range(3))
    module = ox.compile(lambda a, b, c: ((a + b) * c).relu())
    y = module.run(a, b, c)
    assert_bitexact(y.ravel(), oracle.chain_forward(a.ravel(), b.ravel(), c.ravel()), "plan")
    # replay with device-resident inputs: write new inputs into the plan's buffers, replay
    plan = module.plan_for(((4096, 4096),) * 3)
    a2 = r.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    ptr, n = plan.buffer(0)
    stream = plan.stream()
    ox.check(ox.lib().oxh_memcpy_h2d_async(ptr, a2.ctypes.data, n * 4, stream))
    plan.replay()
    out_ptr, m = plan.buffer(plan.plan.output)
    got = np.empty(m, np.float32)
    ox.check(ox.lib().oxh_memcpy_d2h(got.ctypes.data, out_ptr, m * 4, stream))
    assert_bitexact(got, oracle.chain_forward(a2.ravel(), b.ravel(), c.ravel()), "replay")
    plan.close()


def test_graph_capture_error_keeps_stream_usable(module, dev):
    """cuda_graph.rs:84-97: a failed recording ends capture; the stream stays usable."""
    s = torch.cuda.Stream()
    x = torch.ones(16, device=dev)
    y = torch.empty_like(x)
    torch.cuda.synchronize()  # inputs were written on the default stream

    def record_bad():
        module.relu(x, y, stream=s)
        raise ox.OxideError(ox.INVALID_SHAPE, "planted recording failure")

    with pytest.raises(ox.OxideError) as err:
        ox.HipGraphExec.capture(s, record_bad)
    assert err.value.kind == "Execution"
    module.add(x, x, y, stream=s)
    s.synchronize()
    assert host(y).tolist() == [2.0] * 16


def test_graph_replay_of_training_ops_matches_eager(module, dev):
    """BN fwd+bwd, fused CE and AdamW captured once and replayed 4 times with eager work and
    synchronizations between the replays; each replay equals the eager result bit for bit."""
    r = np.random.default_rng(5)
    n, c, h, w = 8, 16, 12, 12
    x = to_dev(r.standard_normal((n, c, h, w)).astype(np.float32), dev)
    gam = to_dev(r.uniform(0.5, 1.5, c).astype(np.float32), dev)
    bet = to_dev(r.uniform(-0.1, 0.1, c).astype(np.float32), dev)
    g = to_dev(r.standard_normal((n, c, h, w)).astype(np.float32), dev)
    logits = to_dev((r.standard_normal((64, 1000)) * 2).astype(np.float32), dev)
    targets = to_dev(r.integers(0, 1000, 64).astype(np.float32), dev)
    p0 = r.standard_normal(5000).astype(np.float32)
    pg = to_dev((r.standard_normal(5000) * 1e-3).astype(np.float32), dev)
    outer = torch.ones(1, device=dev)
    c1, c2 = ox.adamw_corrections(0.9, 0.999, 10)

    def make_state():
        return dict(rm=torch.zeros(c, device=dev), rv=torch.ones(c, device=dev),
                    mean=torch.empty(c, device=dev), inv=torch.empty(c, device=dev),
                    y=torch.empty_like(x), dx=torch.empty_like(x),
                    dw=torch.empty(c, device=dev), db=torch.empty(c, device=dev),
                    loss=torch.empty(1, device=dev), grad=torch.empty_like(logits),
                    p=to_dev(p0, dev), m=torch.zeros(5000, device=dev),
                    v=torch.zeros(5000, device=dev))

    def step(st, mod, stream):
        mod.batch_norm_forward_train(x, gam, bet, st["rm"], st["rv"], st["mean"], st["inv"],
                                     st["y"], stream=stream)
        mod.batch_norm_backward_train(g, x, gam, st["mean"], st["inv"], st["dx"], st["dw"],
                                      st["db"], stream=stream)
        mod.cross_entropy_forward_backward(64, 1000, logits, targets, outer, st["loss"],
                                           st["grad"], stream=stream)
        mod.adamw(1e-3, 0.01, 0.9, 0.999, c1, c2, 1e-8, st["p"], pg, st["m"], st["v"], st["p"],
                  st["m"], st["v"], stream=stream)

    eager = make_state()
    eager_mod = ox.load_kernels(0)
    graphed = make_state()
    graph_mod = ox.load_kernels(0)
    s = torch.cuda.Stream()
    warm = make_state()
    torch.cuda.synchronize()  # states were filled on the default stream
    # one eager step on throw-away state sizes the module's workspaces before capture
    step(warm, graph_mod, s)
    s.synchronize()
    graph = ox.HipGraphExec.capture(s, lambda: step(graphed, graph_mod, s))
    for replay in range(4):
        step(eager, eager_mod, None)
        torch.cuda.synchronize()
        graph.launch(s)
        s.synchronize()
        _ = torch.randn(1000, device=dev).sum().item()  # unrelated eager work between replays
        for k in eager:
            assert torch.equal(eager[k], graphed[k]), (replay, k)


def test_kernel_timer_brackets_one_dispatch(module, dev):
    """oxh_time_next_launch: the armed launch records its own start / stop events; the next
    launch is not timed."""
    x = torch.randn(1 << 24, device=dev)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    t = ox.KernelTimer()
    t.arm()
    module.relu(x, y)
    ms = t.elapsed_ms()
    assert 0.0 < ms < 50.0
    module.relu(x, y)  # not armed: the timer keeps its first interval
    torch.cuda.synchronize()
    assert t.elapsed_ms() == ms
    assert torch.equal(y, torch.relu(x))
