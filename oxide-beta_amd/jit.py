"""The reference's JIT (crates/oxide-torch/src/jit.rs) on liboxide_hip: ``trace`` /
``compile`` record a lazy graph (tensor.py) from placeholders shaped like example inputs; the
first ``run`` for an input signature compiles a plan and caches it (jit.rs:89-176).

* ``lower`` is ``PlanBuilder::lower`` (jit.rs:276-412): one buffer per node (inputs, constants,
  workspaces), Add / Mul / Relu operations, Reshape as an alias of its input's buffer
  (jit.rs:345).  A graph with any other op lowers to no plan (``supported = false``,
  jit.rs:405-408).
* ``HipJitPlan`` is ``CudaJitPlan`` (cuda/jit.rs:10-99) on the library's plan runtime: buffers
  on the device, dependent runs of operations fused into one kernel, the launch list captured
  in a hipGraph and replayed per run between the input and output copies.
* ``EagerPlan`` is ``CompiledPlan::Eager`` (jit.rs:205-207, run_eager 226-243): the traced graph
  evaluated on the device by a forward program, with the placeholders bound to the run's inputs
  (batch statistics recomputed on every run, for instance).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Callable, Sequence

import numpy as np

import oxide_hip as ox
import tensor as tn
from oxide_hip import PLAN_ADD, PLAN_MUL, PLAN_RELU, TRACE, OxideError, check, lib

_u32, _u64, _vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p


@dataclass
class Input:
    elements: int


@dataclass
class Constant:
    values: Sequence[float]


@dataclass
class WorkspaceBuffer:
    elements: int


@dataclass
class Operation:
    op: int
    inputs: tuple[int, ...]
    output: int


@dataclass
class GraphPlan:
    """jit.rs:24-56: buffers, operations, input slots, output slot."""

    buffers: list = field(default_factory=list)
    operations: list[Operation] = field(default_factory=list)
    inputs: list[int] = field(default_factory=list)
    output: int = -1


class HipJitPlan:
    """``CudaJitPlan`` (cuda/jit.rs:10-99) on liboxide_hip's plan runtime."""

    def __init__(self, plan: GraphPlan, device: int = 0):
        import numpy as np

        handle = _vp()
        check(lib().oxh_plan_create(device, ctypes.byref(handle)))
        self._handle = handle.value
        self._slots: list[int] = []
        self._input_slots: list[int] = []
        try:
            for buf in plan.buffers:
                slot = _u32()
                if isinstance(buf, Input):
                    check(lib().oxh_plan_add_input(self._handle, buf.elements,
                                                   ctypes.byref(slot)))
                    self._input_slots.append(len(self._slots))
                elif isinstance(buf, Constant):
                    arr = np.ascontiguousarray(buf.values, dtype=np.float32)
                    check(lib().oxh_plan_add_constant(self._handle, arr.ctypes.data, arr.size,
                                                      ctypes.byref(slot)))
                else:
                    check(lib().oxh_plan_add_workspace(self._handle, buf.elements,
                                                       ctypes.byref(slot)))
                self._slots.append(slot.value)
            if [self._input_slots[i] for i in range(len(self._input_slots))] != list(
                    plan.inputs):
                raise OxideError(TRACE, "plan inputs must be the Input buffers in order")
            for op in plan.operations:
                ins = (_u32 * len(op.inputs))(*[self._slots[i] for i in op.inputs])
                check(lib().oxh_plan_add_operation(self._handle, op.op, ins, len(op.inputs),
                                                   self._slots[op.output]))
            check(lib().oxh_plan_set_output(self._handle, self._slots[plan.output]))
            check(lib().oxh_plan_compile(self._handle))
        except Exception:
            lib().oxh_plan_destroy(self._handle)
            self._handle = None
            raise
        elements = _u64()
        ptr = _vp()
        check(lib().oxh_plan_buffer(self._handle, self._slots[plan.output], ctypes.byref(ptr),
                                    ctypes.byref(elements)))
        self.output_elements = elements.value
        self.plan = plan

    def run(self, inputs: Sequence) -> "np.ndarray":  # noqa: F821
        """H2D inputs, one replay, synchronous D2H of the output (cuda/jit.rs:70-99)."""
        import numpy as np

        arrays = [np.ascontiguousarray(x, dtype=np.float32) for x in inputs]
        ptrs = (_vp * len(arrays))(*[a.ctypes.data for a in arrays])
        out = np.empty(self.output_elements, dtype=np.float32)
        check(lib().oxh_plan_run(self._handle, ptrs, len(arrays), out.ctypes.data, out.size))
        return out

    def replay(self) -> None:
        """One launch of the plan's hipGraph."""
        check(lib().oxh_plan_replay(self._handle))

    def launch(self) -> None:
        """The graph's kernel launches issued directly (no graph launch)."""
        check(lib().oxh_plan_launch(self._handle))

    def stream(self) -> int:
        s = _vp()
        check(lib().oxh_plan_stream(self._handle, ctypes.byref(s)))
        return s.value or 0

    def buffer(self, index: int) -> tuple[int, int]:
        """(device address, elements) of the plan's buffer ``index``."""
        ptr, n = _vp(), _u64()
        check(lib().oxh_plan_buffer(self._handle, self._slots[index], ctypes.byref(ptr),
                                    ctypes.byref(n)))
        return ptr.value, n.value

    def close(self) -> None:
        if self._handle is not None:
            check(lib().oxh_plan_destroy(self._handle))
            self._handle = None

    def __del__(self):
        if getattr(self, "_handle", None) is not None and ox._lib is not None:
            ox._lib.oxh_plan_destroy(self._handle)
            self._handle = None


def lower(output: tn.Tensor, inputs: Sequence[tn.Tensor]):
    """``GraphPlan::compile`` / ``PlanBuilder::lower`` (jit.rs:246-412): the plan, or None when
    the graph holds an op plans do not take (the caller then runs it eagerly)."""
    plan = GraphPlan()
    slots: dict[int, int] = {}
    opcode = {"add": PLAN_ADD, "mul": PLAN_MUL, "relu": PLAN_RELU}
    # Inputs become the first buffers so their slots follow the argument order.
    for p in inputs:
        slots[p.id] = len(plan.buffers)
        plan.buffers.append(Input(p.numel()))
    supported = True
    for node in tn.postorder([output]):
        if node.id in slots:
            continue
        if node.kind == "input":
            raise OxideError(TRACE, "traced graph reads a placeholder that is not an input")
        if node.kind == "constant":
            slots[node.id] = len(plan.buffers)
            plan.buffers.append(Constant(node.value))
        elif node.kind == "parameter":  # a model's parameters are plan constants
            slots[node.id] = len(plan.buffers)
            plan.buffers.append(Constant(node.attrs["param"].host().ravel()))
        elif node.kind == "reshape":
            slots[node.id] = slots[node.args[0].id]
        elif node.kind in opcode:
            args = tuple(slots[a.id] for a in node.args)
            slots[node.id] = len(plan.buffers)
            plan.buffers.append(WorkspaceBuffer(node.numel()))
            plan.operations.append(Operation(opcode[node.kind], args, slots[node.id]))
        else:
            supported = False
            slots[node.id] = len(plan.buffers)
            plan.buffers.append(WorkspaceBuffer(node.numel()))
    if not supported:
        return None
    plan.output = slots[output.id]
    used = {plan.output}
    for op in plan.operations:
        used.update(op.inputs)
    for i, p in enumerate(inputs):
        if slots[p.id] not in used:
            raise OxideError(TRACE, f"traced input {i} is unused")  # jit.rs:259-266
    plan.inputs = [slots[p.id] for p in inputs]
    return plan


class EagerPlan:
    """``CompiledPlan::Eager``: the traced graph evaluated on the device by a forward program
    (tensor.forward_program), the placeholders fed per run."""

    def __init__(self, output: tn.Tensor, placeholders: Sequence[tn.Tensor]):
        self.output, self.placeholders = output, list(placeholders)
        self.program = tn.forward_program(output, self.placeholders)

    def run(self, inputs: Sequence) -> np.ndarray:
        if len(inputs) != len(self.placeholders):
            raise OxideError(TRACE, f"expected {len(self.placeholders)} inputs, "
                                    f"got {len(inputs)}")
        for p, x in zip(self.placeholders, inputs):
            self.program.feed(p, np.ascontiguousarray(x, np.float32).reshape(p.shape))
        self.program.run()
        self.program.check()
        return self.program.value(self.output).host().ravel()


class JitModule:
    """``JitModule`` (jit.rs:14-176): the traced graph, its example input shapes, and one
    compiled plan per input signature."""

    def __init__(self, output: tn.Tensor, placeholders: Sequence[tn.Tensor], device: int = 0):
        self.graph, self.placeholders, self.device = output, list(placeholders), device
        self.input_shapes = [p.shape for p in self.placeholders]
        self._plans: dict[tuple, object] = {}

    def cached_specializations(self) -> int:
        return len(self._plans)

    def output_shape(self) -> tuple:
        return self.graph.shape

    def _validate(self, arrays) -> None:  # jit.rs:183-203
        if len(arrays) != len(self.input_shapes):
            raise OxideError(TRACE, f"expected {len(self.input_shapes)} inputs, got "
                                    f"{len(arrays)}")
        for i, (a, shape) in enumerate(zip(arrays, self.input_shapes)):
            if a.shape != shape:
                raise OxideError(TRACE, f"input {i} expected shape {list(shape)}, got "
                                        f"{list(a.shape)}")

    def plan_for(self, shapes: tuple):
        """The compiled plan of this signature (compile_plan, jit.rs:205-225)."""
        if shapes not in self._plans:
            plan = lower(self.graph, self.placeholders)
            self._plans[shapes] = (HipJitPlan(plan, self.device) if plan is not None
                                   else EagerPlan(self.graph, self.placeholders))
        return self._plans[shapes]

    def run(self, inputs: Sequence) -> np.ndarray:
        arrays = [np.ascontiguousarray(x, dtype=np.float32) for x in inputs]
        self._validate(arrays)
        plan = self.plan_for(tuple(a.shape for a in arrays))
        return plan.run(arrays).reshape(self.graph.shape)


def trace(examples: Sequence, function: Callable) -> JitModule:
    """``jit::trace`` (jit.rs:89-120): ``function`` receives placeholders shaped like
    ``examples`` and returns the traced output."""
    if len(examples) == 0:
        raise OxideError(TRACE, "at least one example input is required")
    placeholders = [tn.input(np.shape(e)) for e in examples]
    output = function(placeholders)
    return JitModule(output, placeholders)


def compile(model: Callable, example) -> JitModule:  # noqa: A001 - mirrors jit::compile
    """``jit::compile`` (jit.rs:131-135): trace ``model``'s forward on one example; its
    parameters become plan constants."""
    return trace([example], lambda inputs: model(inputs[0]))
