"""JIT plans and graph replay on the GPU: the reference's trace / compile KATs (jit.rs:721-761),
config 1's relu((a+b)*c) plan at [4096, 4096] against the oracle, and captured batch-norm /
cross-entropy / AdamW sequences replayed several times with eager work in between, every replay
checked against the eager result."""

import numpy as np
import pytest
import torch

import jit
import oracle
import oxide_hip as ox
import tensor as tn
from helpers import assert_bitexact, host, to_dev

pytestmark = pytest.mark.gpu


def test_trace_caches_and_reuses_a_graph():
    """jit.rs:721-736: trace(x + bias).relu() with x = [-2, 3], bias = ones -> [0, 4]; the plan
    is compiled on the first run and reused."""
    x, bias = np.array([-2.0, 3.0], np.float32), np.ones(2, np.float32)
    module = jit.trace([x, bias], lambda inputs: inputs[0].add(inputs[1]).relu())
    assert module.cached_specializations() == 0
    assert module.run([x, bias]).tolist() == [0.0, 4.0]
    assert module.cached_specializations() == 1
    assert module.run([np.array([5.0, -7.0], np.float32), bias]).tolist() == [6.0, 0.0]
    assert module.cached_specializations() == 1
    assert isinstance(module.plan_for(((2,), (2,))), jit.HipJitPlan)



class _AffineRelu:
    """relu(x * weight + bias) over equal shapes with weight and bias as parameters: the
    reference's compile KAT model (jit.rs:706-719) with its matmul, which is outside this
    path, replaced by the elementwise product."""

    def __init__(self, weight, bias):
        import nn

        self.weight, self.bias = nn.Parameter(weight), nn.Parameter(bias)

    def __call__(self, x):
        return x.mul(self.weight.tensor()).add(self.bias.tensor()).relu()


def test_compile_user_module_parameters_become_plan_constants():
    """jit.rs:131-135, 738-761 (compiles_a_user_defined_module_and_reuses_fixed_workspace):
    compile traces the module's forward on one example; its parameters become Constant buffers
    of the plan, holding their values; two runs on other inputs reuse the one compiled plan and
    its fixed buffers, giving [3, 2] then [0, 0]; one specialisation remains."""
    weight, bias = np.array([[2.0, 3.0]], np.float32), np.array([[1.0, -1.0]], np.float32)
    model = _AffineRelu(weight, bias)
    compiled = jit.compile(model, np.zeros((1, 2), np.float32))
    assert compiled.cached_specializations() == 0
    lowered = jit.lower(compiled.graph, compiled.placeholders)
    kinds = [type(b).__name__ for b in lowered.buffers]
    assert kinds == ["Input", "Constant", "WorkspaceBuffer", "Constant", "WorkspaceBuffer",
                     "WorkspaceBuffer"], kinds
    assert [list(b.values) for b in lowered.buffers if isinstance(b, jit.Constant)] == \
        [[2.0, 3.0], [1.0, -1.0]]
    assert [(o.op, o.inputs, o.output) for o in lowered.operations] == \
        [(ox.PLAN_MUL, (0, 1), 2), (ox.PLAN_ADD, (2, 3), 4), (ox.PLAN_RELU, (4,), 5)]
    first = compiled.run([np.array([[1.0, 1.0]], np.float32)])
    plan = compiled.plan_for(((1, 2),))
    assert isinstance(plan, jit.HipJitPlan)
    buffers = [plan.buffer(i) for i in range(len(plan.plan.buffers))]
    second = compiled.run([np.array([[-1.0, -1.0]], np.float32)])
    assert first.tolist() == [[3.0, 2.0]]
    assert second.tolist() == [[0.0, 0.0]]
    assert compiled.cached_specializations() == 1
    assert compiled.plan_for(((1, 2),)) is plan
    assert [plan.buffer(i) for i in range(len(plan.plan.buffers))] == buffers
    # the constants were taken at compile time: a later change of the parameter is not seen
    # by the compiled plan (its values were copied into the plan's own buffers)
    model.weight.data.fill_(100.0)
    assert compiled.run([np.array([[1.0, 1.0]], np.float32)]).tolist() == [[3.0, 2.0]]


def test_compile_user_module_matches_oracle_on_ragged_shape():
    """The compiled relu(x * w + b) on [257, 1031] (not a multiple of the float4 width) with
    random parameters, run on two inputs: bit-exact against the oracle's add / mul / relu
    (evaluation.rs:21-34) each time, one specialisation."""
    r = np.random.default_rng(0x6F78696400000011)
    shape = (257, 1031)
    weight, bias = (r.uniform(-1, 1, shape).astype(np.float32) for _ in range(2))
    compiled = jit.compile(_AffineRelu(weight, bias), np.zeros(shape, np.float32))
    for _ in range(2):
        x = r.uniform(-1, 1, shape).astype(np.float32)
        ref = oracle.relu(oracle.add(oracle.mul(x.ravel(), weight.ravel()), bias.ravel()))
        assert_bitexact(compiled.run([x]).ravel(), ref, "compiled module")
    assert compiled.cached_specializations() == 1

def test_run_validates_inputs_like_reference():
    """jit.rs:183-203: input count and shape must match the trace (Error::Trace)."""
    a = np.array([1, -1], np.float32)
    module = jit.trace([a, a], lambda i: (i[0] * i[1]).relu())
    assert module.run([a, np.array([2, 2], np.float32)]).tolist() == [2.0, 0.0]
    assert module.run([np.array([1, 3], np.float32), np.array([2, 2], np.float32)]).tolist() \
        == [2.0, 6.0]
    for bad in ([a], [a, a, a], [a, np.ones(3, np.float32)]):
        with pytest.raises(ox.OxideError) as err:
            module.run(bad)
        assert err.value.kind == "Trace"
    assert module.cached_specializations() == 1


def test_reshape_in_a_plan_is_an_alias():
    """jit.rs:345: reshape between plan ops costs no buffer and no launch; the output has the
    traced shape."""
    x = np.arange(-3, 3, dtype=np.float32).reshape(2, 3)
    module = jit.trace([x], lambda i: i[0].relu().reshape((3, 2)).mul(
        tn.constant(np.full((3, 2), 2.0))))
    y = module.run([x])
    assert y.shape == (3, 2)
    np.testing.assert_array_equal(y, np.maximum(x, 0).reshape(3, 2) * 2)
    assert isinstance(module.plan_for(((2, 3),)), jit.HipJitPlan)


def test_config1_plan_matches_oracle():
    """Config 1 via compile: relu((a+b)*c), three [4096, 4096] inputs, values U(-1, 1)."""
    r = np.random.default_rng(0x6F78696400000001)
    a, b, c = (r.uniform(-1, 1, (4096, 4096)).astype(np.float32) for _ in range(3))
    module = jit.trace([a, b, c], lambda i: ((i[0] + i[1]) * i[2]).relu())
    y = module.run([a, b, c])
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
    # the same launches issued directly (no graph launch)
    a3 = r.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    ox.check(ox.lib().oxh_memcpy_h2d_async(ptr, a3.ctypes.data, n * 4, stream))
    plan.launch()
    ox.check(ox.lib().oxh_memcpy_d2h(got.ctypes.data, out_ptr, m * 4, stream))
    assert_bitexact(got, oracle.chain_forward(a3.ravel(), b.ravel(), c.ravel()), "launch")
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


def _host_plan(plan, inputs, state=None):
    """The plan evaluated op by op on the host with the oracle's elementwise functions.
    Workspaces start at zero, as the compiled plan's do, and keep their values from one run to
    the next (``state``); returns (output, state)."""
    bufs, k = [], 0
    for i, b in enumerate(plan.buffers):
        if isinstance(b, jit.Input):
            bufs.append(np.asarray(inputs[k], np.float32).ravel())
            k += 1
        elif isinstance(b, jit.Constant):
            bufs.append(np.asarray(b.values, np.float32))
        else:
            bufs.append(state[i] if state is not None else np.zeros(b.elements, np.float32))
    fn = {ox.PLAN_ADD: oracle.add, ox.PLAN_MUL: oracle.mul, ox.PLAN_MUL_BACKWARD: oracle.mul,
          ox.PLAN_ACCUMULATE: oracle.accumulate, ox.PLAN_RELU_BACKWARD: oracle.relu_backward}
    for op in plan.operations:
        args = [bufs[i] for i in op.inputs]
        bufs[op.output] = (oracle.relu(args[0]) if op.op == ox.PLAN_RELU
                           else fn[op.op](args[0], args[1]))
    return bufs[plan.output], bufs


def _plan(n_inputs, n_work, ops, output, elements, constant=None):
    buffers = [jit.Input(elements) for _ in range(n_inputs)]
    if constant is not None:
        buffers.append(jit.Constant(constant))
    buffers += [jit.WorkspaceBuffer(elements) for _ in range(n_work)]
    return jit.GraphPlan(buffers=buffers, operations=[jit.Operation(*o) for o in ops],
                        inputs=list(range(n_inputs)), output=output)


A, M, R, RB, MB, ACC = (ox.PLAN_ADD, ox.PLAN_MUL, ox.PLAN_RELU, ox.PLAN_RELU_BACKWARD,
                        ox.PLAN_MUL_BACKWARD, ox.PLAN_ACCUMULATE)


@pytest.mark.parametrize("name,n_in,n_work,ops,out", [
    # x * x (the running value as both operands), then relu
    ("square", 1, 2, [(M, (0, 0), 1), (R, (1,), 2)], 2),
    # the running value as the second input of a non-commutative op, in both positions
    ("relu_backward_sides", 2, 3, [(A, (0, 1), 2), (RB, (1, 2), 3), (RB, (3, 0), 4)], 4),
    # an intermediate read again after the run: stored, and a new run starts from it
    ("reused_intermediate", 2, 4, [(A, (0, 1), 2), (M, (2, 1), 3), (R, (0,), 4),
                                   (ACC, (2, 4), 5)], 5),
    # the output written in the middle of a run
    ("output_mid_run", 2, 3, [(A, (0, 1), 2), (M, (2, 0), 3), (R, (3,), 4)], 3),
    # a run reading a buffer written earlier in it ends there
    ("reads_earlier_write", 2, 3, [(A, (0, 1), 2), (M, (2, 1), 3), (A, (3, 2), 4)], 4),
    # write-after-read inside a run: op 2 rewrites the buffer op 0 read (the next replay's op 0
    # reads it), once as the output and once as an internal workspace
    ("rewrite_read_buffer", 1, 4, [(A, (0, 2), 3), (MB, (3, 0), 4), (A, (4, 0), 2)], 2),
    ("rewrite_read_internal", 1, 4, [(A, (0, 2), 3), (MB, (3, 0), 2), (A, (2, 0), 4)], 4),
    # longer than one fused run (eight steps), with stores of a buffer written twice
    ("long", 2, 3, [(A, (0, 1), 2), (M, (2, 1), 3), (R, (3,), 2), (A, (2, 0), 3), (M, (3, 3), 4),
                    (ACC, (4, 1), 2), (R, (2,), 3), (A, (3, 0), 4), (M, (4, 1), 2),
                    (RB, (0, 2), 3), (A, (3, 3), 4)], 4),
])
@pytest.mark.parametrize("elements", [4096 * 1024 + 3, 5])
def test_fused_plan_runs_match_op_by_op(name, n_in, n_work, ops, out, elements):
    """Compiled plans fuse runs of dependent operations into one kernel; the output equals the
    op-by-op evaluation with the oracle bit for bit (ragged lengths exercise the tail)."""
    ws = list(range(n_in, n_in + n_work))
    plan = _plan(n_in, n_work, ops, out, elements)
    assert all(o[2] in ws for o in ops)
    r = np.random.default_rng(hash(name) & 0xFFFF)
    inputs = [r.uniform(-1, 1, elements).astype(np.float32) for _ in range(n_in)]
    inputs[0][:3] = [0.0, -0.0, np.nan]
    hp = jit.HipJitPlan(plan)
    state = None
    try:
        for _ in range(3):  # later replays start from the earlier ones' workspaces
            got = hp.run(inputs)
            ref, state = _host_plan(plan, inputs, state)
            assert_bitexact(got, ref, name)
            inputs = [x[::-1].copy() for x in inputs]
    finally:
        hp.close()


@pytest.mark.parametrize("offset,nbytes", [(0, 4), (1, 1), (3, 17), (5, 4093), (16, 4096),
                                           (7, (1 << 20) + 9), (0, 64 << 20)])
def test_memset0_zeroes_exactly_the_range(dev, offset, nbytes):
    """oxh_memset0_async (DeviceBuffer::zeroed, runtime.rs:83-105) at any byte alignment: the
    range becomes zero and the bytes either side keep their values."""
    buf = torch.full((offset + nbytes + 32,), 0xAB, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    ox.check(ox.lib().oxh_memset0_async(buf.data_ptr() + offset, nbytes, ox.current_stream()))
    torch.cuda.synchronize()
    h = host(buf)
    assert (h[:offset] == 0xAB).all()
    assert (h[offset:offset + nbytes] == 0).all()
    assert (h[offset + nbytes:] == 0xAB).all()


def test_memset0_replays_in_a_graph(dev):
    """The zero fill recorded into a graph clears the buffer again on every replay, with eager
    writes to it between the replays."""
    s = torch.cuda.Stream()
    buf = torch.ones(100003, device=dev)
    torch.cuda.synchronize()
    graph = ox.HipGraphExec.capture(
        s, lambda: ox.check(ox.lib().oxh_memset0_async(buf.data_ptr() + 4, 4 * 100000,
                                                       s.cuda_stream)))
    for replay in range(4):
        buf.fill_(float(replay + 2))
        torch.cuda.synchronize()
        graph.launch(s)
        s.synchronize()
        h = host(buf)
        assert h[0] == replay + 2 and (h[1:100001] == 0).all() and (h[100001:] == replay + 2).all()
