"""CPU-side checks of the C ABI: the library loads and exports every declared symbol, and the
host logic (argument validation, workspace sizing, AdamW corrections, plan building, trace
lowering) behaves like the reference.  No call here reaches a GPU: every failing call is
rejected on the host before any launch."""

import ctypes

import numpy as np
import pytest

import jit
import oracle
import oxide_hip as ox
import tensor as tn


def test_library_exports_every_header_symbol():
    lib = ox.lib()
    symbols = ox.header_symbols()
    assert len(symbols) >= 50
    missing = [s for s in symbols if not hasattr(lib, s)]
    assert not missing, missing
    # every declared function also has a ctypes signature in the front ends
    import tensor
    import training

    bound = set(ox._SIGNATURES) | set(training.signatures()) | set(tensor.signatures())
    assert set(symbols) <= bound, set(symbols) - bound
    assert ox.lib().oxh_version().decode().startswith("oxide-hip")


def test_integration_guide_names_every_header_function():
    """The binding guide's function table stays in step with the header."""
    guide = (ox.HEADER_PATH.parent.parent / "INTEGRATION.md").read_text()
    missing = [s for s in ox.header_symbols() if f"`{s}`" not in guide and f"{s}(" not in guide]
    assert not missing, missing


def _status(call):
    return call


def test_elementwise_rejects_null_and_partial_overlap():
    lib = ox.lib()
    assert lib.oxh_add(None, None, 16, 32, 4) == ox.INVALID_SHAPE
    assert b"null" in lib.oxh_last_error()
    # output overlapping an input by a partial offset is refused (exact aliasing is allowed)
    base = 1 << 20
    assert lib.oxh_add(None, base, base + 4096, base + 4, 100) == ox.INVALID_SHAPE
    assert b"overlap" in lib.oxh_last_error()
    # n == 0 is a no-op that touches nothing
    assert lib.oxh_add(None, None, None, None, 0) == ox.OK
    # chain backward outputs must be distinct
    assert lib.oxh_elementwise_chain_backward(None, 16, 32, 48, None, 1 << 20, 1 << 20,
                                              1 << 21, 8) == ox.INVALID_SHAPE


def test_batch_norm_rejects_single_sample_like_reference():
    """evaluation.rs:498-502 / runtime.rs:543-547: Error::Execution."""
    lib = ox.lib()
    ws = ctypes.c_uint64()
    assert lib.oxh_batch_norm_workspace_size(1, 2, 1, ctypes.byref(ws)) == ox.OK
    st = lib.oxh_batch_norm_statistics(None, 1, 2, 1, 1e-5, 256, 512, 768, 1024, 4096,
                                       ws.value)
    assert st == ox.EXECUTION
    assert b"more than one value per channel" in lib.oxh_last_error()
    with pytest.raises(oracle.OracleError) as err:
        oracle.bn_forward(np.ones((1, 2, 1, 1), np.float32), np.ones(2, np.float32),
                          np.zeros(2, np.float32), np.zeros(2, np.float32),
                          np.ones(2, np.float32))
    assert err.value.kind == "Execution"


def test_batch_norm_workspace_checks():
    lib = ox.lib()
    size = ox.batch_norm_workspace_size(64, 128, 3136)
    assert size % 256 == 0 and size >= 128 * 16
    # too small a workspace is refused before launch
    st = lib.oxh_batch_norm_statistics(None, 64, 128, 3136, 1e-5, 256, 512, 768, 1024, 4096,
                                       size - 256)
    assert st == ox.INVALID_SHAPE and b"workspace" in lib.oxh_last_error()
    assert ox.batch_norm_workspace_size(1, 1, 2) >= 16
    with pytest.raises(ox.OxideError) as err:
        ox.batch_norm_workspace_size(0, 3, 3)
    assert err.value.kind == "InvalidShape"


def test_cross_entropy_argument_checks():
    lib = ox.lib()
    assert ox.cross_entropy_workspace_size(8192, 32768) >= 8192 * 8
    # the gradient needs the upstream scalar
    st = lib.oxh_cross_entropy_backward(None, 2, 3, 256, 512, None, 4096, None)
    assert st == ox.INVALID_SHAPE
    # empty logits
    assert lib.oxh_cross_entropy_backward(None, 0, 3, 256, 512, 768, 4096, None) == \
        ox.INVALID_SHAPE


@pytest.mark.parametrize("step", [1, 2, 3, 7, 10, 100, 1000, 65537])
def test_adamw_corrections_match_reference_powi(step):
    """optim.rs:91-92 / 113-114: 1 - beta.powi(step) with compiler-rt's __powisf2."""
    c1, c2 = ox.adamw_corrections(0.9, 0.999, step)
    assert np.float32(c1) == np.float32(1.0) - np.float32(oracle.powi(0.9, step))
    assert np.float32(c2) == np.float32(1.0) - np.float32(oracle.powi(0.999, step))


def test_adamw_rejects_non_finite_hyper_parameters():
    lib = ox.lib()
    st = lib.oxh_adamw(None, float("nan"), 0.01, 0.9, 0.999, 0.5, 0.5, 1e-8, 256, 512, 768,
                       1024, 256, 768, 1024, 4)
    assert st == ox.INVALID_SHAPE


def test_plan_builder_validation():
    lib = ox.lib()
    h = ctypes.c_void_p()
    assert lib.oxh_plan_create(0, ctypes.byref(h)) == ox.OK
    a, b, w = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
    assert lib.oxh_plan_add_input(h, 4, ctypes.byref(a)) == ox.OK
    assert lib.oxh_plan_add_input(h, 4, ctypes.byref(b)) == ox.OK
    assert lib.oxh_plan_add_workspace(h, 4, ctypes.byref(w)) == ox.OK
    ins = (ctypes.c_uint32 * 2)(a.value, b.value)
    # wrong arity, unknown op, writing an input, reading own output, size mismatch
    assert lib.oxh_plan_add_operation(h, ox.PLAN_RELU, ins, 2, w.value) == ox.TRACE
    assert lib.oxh_plan_add_operation(h, 99, ins, 2, w.value) == ox.TRACE
    assert lib.oxh_plan_add_operation(h, ox.PLAN_ADD, ins, 2, a.value) == ox.TRACE
    self_read = (ctypes.c_uint32 * 2)(a.value, w.value)
    assert lib.oxh_plan_add_operation(h, ox.PLAN_ADD, self_read, 2, w.value) == ox.TRACE
    big = ctypes.c_uint32()
    assert lib.oxh_plan_add_input(h, 8, ctypes.byref(big)) == ox.OK
    mism = (ctypes.c_uint32 * 2)(a.value, big.value)
    assert lib.oxh_plan_add_operation(h, ox.PLAN_ADD, mism, 2, w.value) == ox.INVALID_SHAPE
    assert lib.oxh_plan_add_operation(h, ox.PLAN_ADD, ins, 2, w.value) == ox.OK
    # running an uncompiled plan is a Trace error
    out = np.empty(4, np.float32)
    assert lib.oxh_plan_run(h, None, 0, out.ctypes.data, 4) == ox.TRACE
    assert lib.oxh_plan_replay(h) == ox.TRACE
    assert lib.oxh_plan_destroy(h) == ox.OK


def test_trace_lowering_matches_reference_plan_shape():
    """PlanBuilder::lower (jit.rs:276-412): relu((a + b) * c) -> 3 inputs, 3 workspaces."""
    a, b, c = (tn.input((4096, 4096)) for _ in range(3))
    plan = jit.lower(((a + b) * c).relu(), [a, b, c])
    kinds = [type(x).__name__ for x in plan.buffers]
    assert kinds == ["Input"] * 3 + ["WorkspaceBuffer"] * 3
    assert [o.op for o in plan.operations] == [ox.PLAN_ADD, ox.PLAN_MUL, ox.PLAN_RELU]
    assert plan.operations[0].inputs == (0, 1) and plan.operations[1].inputs == (3, 2)
    assert plan.output == 5 and plan.inputs == [0, 1, 2]


def test_trace_rejects_unused_input_and_shape_mismatch():
    """jit.rs:259-266 (unused traced input) and tensor/mod.rs:536-552 (equal shapes)."""
    a, b = tn.input((2,)), tn.input((2,))
    with pytest.raises(ox.OxideError) as err:
        jit.lower(a.relu(), [a, b])
    assert err.value.kind == "Trace"
    with pytest.raises(ox.OxideError) as err:
        tn.input((2,)) + tn.input((3,))
    assert err.value.kind == "InvalidShape"


def test_trace_constants_become_constant_buffers():
    x = tn.input((2,))
    plan = jit.lower((x + tn.constant([1.0, 1.0])).relu(), [x])
    assert [type(b).__name__ for b in plan.buffers] == ["Input", "Constant", "WorkspaceBuffer",
                                                       "WorkspaceBuffer"]


def test_reshape_lowers_as_an_alias():
    """jit.rs:345: Reshape takes its input's buffer, no operation and no new buffer."""
    x = tn.input((2, 3))
    y = x.relu().reshape((3, 2)).reshape((6,)).relu()
    plan = jit.lower(y, [x])
    assert [type(b).__name__ for b in plan.buffers] == ["Input", "WorkspaceBuffer",
                                                       "WorkspaceBuffer"]
    assert [(o.op, o.inputs, o.output) for o in plan.operations] == [
        (ox.PLAN_RELU, (0,), 1), (ox.PLAN_RELU, (1,), 2)]
    with pytest.raises(ox.OxideError) as err:
        x.reshape((4,))
    assert err.value.kind == "InvalidShape"


def test_graphs_plans_cannot_take_lower_to_no_plan():
    """jit.rs:405-408 (supported = false -> CompiledPlan::Eager): BatchNorm, cross entropy,
    conv and pooling are not plan operations, and an unused input is then no error."""
    x, t = tn.input((2, 3, 1, 2)), tn.input((2,))
    state = tn.BatchNormState.__new__(tn.BatchNormState)
    state.channels = 3
    w, b = tn.constant(np.ones(3)), tn.constant(np.zeros(3))
    y = x.batch_norm2d(w, b, state, True, 0.1, 1e-5).relu()
    assert jit.lower(y, [x]) is None
    assert jit.lower(y.reshape((2, 6)).cross_entropy(t), [x, t]) is None
    assert jit.lower(y.avg_pool2d((1, 2), (1, 2)), [x, tn.input((5,))]) is None


def test_lazy_builders_follow_reference_shape_rules():
    """tensor/mod.rs:158-389: conv2d, avg_pool2d, batch_norm2d and cross_entropy argument
    errors with the reference's kinds."""
    x = tn.input((2, 4, 5, 5))
    w = tn.constant(np.zeros((8, 2, 3, 3)))
    b = tn.constant(np.zeros(8))
    assert x.conv2d(w, b, 2, 1, 2).shape == (2, 8, 3, 3)
    for args in [(tn.constant(np.zeros((8, 2, 3, 2))), b, 1, 1, 2),   # non-square kernel
                 (w, b, 1, 1, 3),                                      # groups
                 (w, tn.constant(np.zeros(7)), 1, 1, 2),               # bias size
                 (w, b, 0, 1, 2)]:                                     # stride 0
        with pytest.raises(ox.OxideError) as err:
            x.conv2d(*args)
        assert err.value.kind == "InvalidShape"
    with pytest.raises(ox.OxideError):
        tn.input((1, 1, 2, 2)).conv2d(tn.constant(np.zeros((1, 1, 5, 5))), tn.constant([0.0]),
                                      1, 1, 1)  # kernel exceeds the padded input
    assert x.avg_pool2d((2, 3), (2, 1)).shape == (2, 4, 2, 3)
    assert x.global_avg_pool2d().shape == (2, 4, 1, 1)
    with pytest.raises(ox.OxideError):
        x.avg_pool2d((6, 1), (1, 1))
    state = tn.BatchNormState.__new__(tn.BatchNormState)
    state.channels = 4
    ones = tn.constant(np.ones(4))
    for m, e in [(1.5, 1e-5), (float("nan"), 1e-5), (0.1, 0.0), (0.1, float("inf"))]:
        with pytest.raises(ox.OxideError) as err:
            x.batch_norm2d(ones, ones, state, True, m, e)
        assert err.value.kind == "Execution"
    with pytest.raises(ox.OxideError) as err:
        tn.input((2, 3)).cross_entropy(tn.input((3,)))
    assert err.value.kind == "InvalidShape"


def test_net_builders_check_shapes_on_the_host():
    """oxh_net_* validation (no device work): the same rules in the C ABI."""
    import ctypes

    import tensor

    L = tensor._lib()
    h = ctypes.c_void_p()
    assert L.oxh_net_create(ctypes.byref(h)) == ox.OK
    u32 = ctypes.c_uint32
    node = lambda: u32()  # noqa: E731
    shape = lambda *d: (ctypes.c_uint64 * len(d))(*d)  # noqa: E731
    x, w, b, t, r = node(), node(), node(), node(), node()
    assert L.oxh_net_input(h, 4, shape(2, 3, 4, 4), 0, ctypes.byref(x)) == ox.OK
    assert L.oxh_net_parameter(h, 4, shape(5, 3, 3, 3), 4096, ctypes.byref(w)) == ox.OK
    assert L.oxh_net_parameter(h, 1, shape(5), 8192, ctypes.byref(b)) == ox.OK
    assert L.oxh_net_conv2d(h, x.value, w.value, b.value, 1, 1, 1, ctypes.byref(r)) == ox.OK
    rank, dims = u32(), (ctypes.c_uint64 * 4)()
    assert L.oxh_net_node_shape(h, r.value, ctypes.byref(rank), dims) == ox.OK
    assert rank.value == 4 and list(dims) == [2, 5, 4, 4]
    assert L.oxh_net_conv2d(h, x.value, w.value, b.value, 1, 1, 2, ctypes.byref(r)) == \
        ox.INVALID_SHAPE
    assert L.oxh_net_add(h, x.value, r.value, ctypes.byref(t)) == ox.INVALID_SHAPE
    assert L.oxh_net_input(h, 0, shape(1), 0, ctypes.byref(t)) == ox.INVALID_SHAPE
    assert b"scalar" in L.oxh_last_error()
    assert L.oxh_net_batch_norm2d(h, r.value, b.value, b.value, 256, 512, 1, 0.1, 0.0,
                                  ctypes.byref(t)) == ox.EXECUTION
    assert L.oxh_net_reshape(h, r.value, 2, shape(10, 17), ctypes.byref(t)) == ox.INVALID_SHAPE
    assert L.oxh_net_relu(h, 999, ctypes.byref(t)) == ox.INVALID_SHAPE
    # a training program needs a one-element root (tensor/mod.rs:399-404), checked before
    # anything is allocated
    prog = ctypes.c_void_p()
    assert L.oxh_net_training_program(h, r.value, None, ctypes.byref(prog)) == ox.EXECUTION
    assert b"scalar" in L.oxh_last_error()
    assert L.oxh_net_destroy(h) == ox.OK


def test_conv_forward_order_query():
    """oxh_conv2d_forward_serial: the forwards that would leave most of the chip idle sum four
    ordered parts (the MNIST MobileNetV4's long-channel 1x1 layers on 1x1 planes, the fused
    blocks' 3x3 convolutions); the stem, short-channel and large-grid forwards stay serial."""
    sh = ox.conv2d_shape
    assert ox.conv2d_forward_serial(sh(128, 1, 28, 28, 32, 3, 2, 1, 1))        # stem
    assert not ox.conv2d_forward_serial(sh(128, 32, 14, 14, 32, 3, 2, 1, 1))   # 7x7 output
    assert not ox.conv2d_forward_serial(sh(128, 32, 7, 7, 96, 3, 2, 1, 1))     # 4x4 output
    assert not ox.conv2d_forward_serial(sh(128, 512, 1, 1, 128, 1, 1, 0, 1))   # UIB project
    assert ox.conv2d_forward_serial(sh(128, 128, 1, 1, 512, 1, 1, 0, 1))       # 128 channels
    assert ox.conv2d_forward_serial(sh(128, 64, 8, 8, 256, 1, 1, 0, 1))        # large grid
    assert ox.conv2d_forward_serial(sh(2, 8, 5, 5, 8, 3, 1, 1, 8))             # grouped
    with pytest.raises(ox.OxideError):
        ox.conv2d_forward_serial(sh(1, 1, 1, 1, 1, 3, 1, 0, 1))                # kernel > input


def test_conv_input_gradient_order_query():
    """oxh_conv2d_input_backward_serial: a pointwise input gradient over at least 256 output
    channels on a grid that leaves the chip waiting on its serial chains (the MNIST
    MobileNetV4's head, its 1x1-plane expands and the 960-channel conv) sums four ordered parts,
    and a stride-2 K x K one (the fused blocks') sums on the matrix cores; short channel sums,
    large grids, stride-1 and grouped K x K kernels stay serial."""
    sh = ox.conv2d_shape
    assert not ox.conv2d_input_backward_serial(sh(128, 960, 1, 1, 1280, 1, 1, 0, 1))  # head
    assert not ox.conv2d_input_backward_serial(sh(128, 128, 1, 1, 960, 1, 1, 0, 1))
    assert not ox.conv2d_input_backward_serial(sh(128, 128, 1, 1, 512, 1, 1, 0, 1))   # expand
    assert ox.conv2d_input_backward_serial(sh(128, 512, 1, 1, 128, 1, 1, 0, 1))       # project
    assert ox.conv2d_input_backward_serial(sh(128, 1280, 1, 1, 10, 1, 1, 0, 1))       # classifier
    assert ox.conv2d_input_backward_serial(sh(128, 64, 8, 8, 256, 1, 1, 0, 1))        # large grid
    assert not ox.conv2d_input_backward_serial(sh(128, 32, 7, 7, 96, 3, 2, 1, 1))     # stride 2
    assert ox.conv2d_input_backward_serial(sh(2, 18, 6, 6, 20, 3, 1, 1, 1))           # stride 1
    assert ox.conv2d_input_backward_serial(sh(2, 8, 5, 5, 8, 3, 2, 1, 8))             # grouped
    with pytest.raises(ox.OxideError):
        ox.conv2d_input_backward_serial(sh(1, 1, 1, 1, 1, 3, 1, 0, 1))


def test_conv_backward_rejects_an_overlapping_addend():
    """oxh_conv2d_backward forms the input and weight gradients in one launch: the addend it
    reads may be input_gradient itself, never a part of it, nor any other buffer the launch
    writes.  oxh_conv2d_input_backward_accumulate takes the same rule.  Host checks only (the
    pointers are never dereferenced)."""
    lib = ox.lib()
    shape = ox.conv2d_shape(2, 8, 4, 4, 16, 1, 1, 0, 1)
    ws = ox.conv2d_workspace_size(shape)
    nx, ny, nw = 2 * 8 * 16 * 4, 2 * 16 * 16 * 4, 16 * 8 * 4
    base = 1 << 24
    g, x, w = base, base + (1 << 16), base + (2 << 16)
    dx, dw, db, wsp = base + (3 << 16), base + (4 << 16), base + (5 << 16), base + (6 << 16)
    assert nx < (1 << 16) and ny < (1 << 16) and nw < (1 << 16) and ws < (1 << 16)

    def backward(addend, bias=db):
        return lib.oxh_conv2d_backward(None, ctypes.byref(shape), g, x, w, addend, dx, dw, bias,
                                       wsp if ws else None, ws)

    for bad in (dx + 4, dw, dw - nx + 4, db - 4, wsp):
        if bad == wsp and ws == 0:
            continue
        assert backward(bad) == ox.INVALID_SHAPE, hex(bad)
        assert b"overlap" in lib.oxh_last_error()
    # a partial overlap with input_gradient is refused by the accumulate entry point too
    assert lib.oxh_conv2d_input_backward_accumulate(None, ctypes.byref(shape), g, w, dx + 4,
                                                    dx) == ox.INVALID_SHAPE
    assert b"partially overlaps" in lib.oxh_last_error()
    assert lib.oxh_conv2d_input_backward_accumulate(None, ctypes.byref(shape), g, w, x,
                                                    g) == ox.INVALID_SHAPE
    assert b"overlaps an operand" in lib.oxh_last_error()
