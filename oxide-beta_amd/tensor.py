"""The lazy tensor graph of oxide-torch on the MI355X: the reference's ``Tensor`` builders with
their shape rules (crates/oxide-torch/src/tensor/mod.rs:103-389; graph.rs:70-139), lowered to a
liboxide_hip net (``oxh_net_*``) and run as device programs (``oxh_program_*``):

* ``forward_program(output)`` -- the eager device evaluation of a node (runtime.rs:125-379),
  which is also what a JIT plan the fused-plan compiler cannot take runs (jit.rs:205-243);
* ``training_program(loss, adamw)`` -- forward, reverse mode from a one-element root
  (``Tensor::backward``, tensor/mod.rs:399-422 -> runtime.rs:1198-1217) and optionally one
  AdamW step over every parameter the loss reaches (optim.rs:78-152).

A ``Program`` exposes each node's value and gradient buffer (``Tensor::grad``,
tensor/mod.rs:429-444), runs eagerly or from one captured hipGraph, and lists its launch groups
(``training.Op``) so each can be checked against the oracle.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

import oxide_hip as ox
import training as T

_u32, _u64, _vp, _f32, _int = (ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p,
                               ctypes.c_float, ctypes.c_int)


class AdamWConfig(ctypes.Structure):
    _fields_ = [("learning_rate", _f32), ("weight_decay", _f32), ("beta1", _f32),
                ("beta2", _f32), ("epsilon", _f32)]


_P = ctypes.POINTER
_SIGNATURES = {
    "oxh_net_create": [_P(_vp)],
    "oxh_net_destroy": [_vp],
    "oxh_net_node_count": [_vp, _P(_u32)],
    "oxh_net_node_shape": [_vp, _u32, _P(_u32), _u64 * 4],
    "oxh_net_input": [_vp, _u32, _P(_u64), _int, _P(_u32)],
    "oxh_net_parameter": [_vp, _u32, _P(_u64), _vp, _P(_u32)],
    "oxh_net_constant": [_vp, _u32, _P(_u64), _vp, _P(_u32)],
    "oxh_net_add": [_vp, _u32, _u32, _P(_u32)],
    "oxh_net_mul": [_vp, _u32, _u32, _P(_u32)],
    "oxh_net_relu": [_vp, _u32, _P(_u32)],
    "oxh_net_reshape": [_vp, _u32, _u32, _P(_u64), _P(_u32)],
    "oxh_net_conv2d": [_vp, _u32, _u32, _u32, _u64, _u64, _u64, _P(_u32)],
    "oxh_net_avg_pool2d": [_vp, _u32, _u64, _u64, _u64, _u64, _P(_u32)],
    "oxh_net_batch_norm2d": [_vp, _u32, _u32, _u32, _vp, _vp, _int, _f32, _f32, _P(_u32)],
    "oxh_net_cross_entropy": [_vp, _u32, _u32, _P(_u32)],
    "oxh_net_forward_program": [_vp, _u32, _P(_vp)],
    "oxh_net_training_program": [_vp, _u32, _P(AdamWConfig), _P(_vp)],
    "oxh_program_value": [_vp, _u32, _P(_vp)],
    "oxh_program_gradient": [_vp, _u32, _P(_vp)],
    "oxh_program_destroy": [_vp],
    "oxh_program_check": [_vp],
    "oxh_program_steps": [_vp, _P(ctypes.c_int32)],
}
_bound = None


def _lib():
    global _bound
    if _bound is None:
        handle = T._lib()  # the program inspection entry points are typed there
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        _bound = handle
    return _bound


def _call(name, *args):
    ox.check(getattr(_lib(), name)(*args))


def signatures() -> dict:
    return dict(_SIGNATURES)


def _err(kind: int, message: str) -> ox.OxideError:
    return ox.OxideError(kind, message)


# ----------------------------------------------------------------------------- lazy graph

class BatchNormState:
    """Running statistics of a BatchNorm2d (graph.rs:47-54): device vectors, mean 0 and
    variance 1 at creation (nn.rs:139-140), updated in place by training-mode forwards."""

    def __init__(self, channels: int, running_mean=None, running_variance=None):
        import torch

        self.channels = int(channels)
        dev = torch.device("cuda:0") if torch.cuda.is_available() else torch.device("cpu")
        self.running_mean = (torch.zeros(self.channels, device=dev) if running_mean is None
                             else running_mean)
        self.running_variance = (torch.ones(self.channels, device=dev)
                                 if running_variance is None else running_variance)


class Tensor:
    """A traced value: a leaf (``input``, ``constant``, ``parameter``) or an op of traced
    values.  Builders validate as tensor/mod.rs does and raise ``OxideError`` of the same
    kind; nothing runs until a program is built and run."""

    _next_id = 0

    def __init__(self, shape, kind, args=(), value=None, **attrs):
        self.shape = tuple(int(s) for s in shape)
        self.kind = kind
        self.args = tuple(args)
        self.value = value  # constant: host values
        self.attrs = attrs
        Tensor._next_id += 1
        self.id = Tensor._next_id

    def __repr__(self):
        return f"Tensor({self.kind}, {self.shape})"

    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def requires_grad(self) -> bool:
        return self.kind == "parameter" or bool(self.attrs.get("requires_grad", False))

    # -- elementwise (tensor/mod.rs:103-122, 536-552)
    def _binary(self, other, kind):
        if not isinstance(other, Tensor):
            other = constant(other, self.shape)
        if other.shape != self.shape:
            raise _err(ox.INVALID_SHAPE,
                       f"elementwise operands differ: {list(self.shape)} and {list(other.shape)}")
        return Tensor(self.shape, kind, (self, other))

    def add(self, other):
        return self._binary(other, "add")

    def mul(self, other):
        return self._binary(other, "mul")

    def relu(self):
        return Tensor(self.shape, "relu", (self,))

    __add__ = add
    __mul__ = mul

    # tensor/mod.rs:125-150: built lazily, but no device kernel serves it on this path
    def matmul(self, other):
        if len(self.shape) != 2 or len(other.shape) != 2:
            raise _err(ox.INVALID_SHAPE, "matmul expects two rank-2 tensors")
        if self.shape[1] != other.shape[0]:
            raise _err(ox.INVALID_SHAPE, "matmul dimensions do not align")
        return Tensor((self.shape[0], other.shape[1]), "matmul", (self, other))

    # tensor/mod.rs:293-301
    def reshape(self, shape):
        shape = tuple(int(s) for s in shape)
        if not shape:
            raise _err(ox.INVALID_SHAPE, "scalar shapes are not implemented")
        n = 1
        for s in shape:
            n *= s
        if n != self.numel():
            raise _err(ox.INVALID_SHAPE, "reshape must preserve the element count")
        return Tensor(shape, "reshape", (self,))

    # tensor/mod.rs:158-237
    def conv2d(self, weight, bias, stride: int, padding: int, groups: int):
        if len(self.shape) != 4 or len(weight.shape) != 4 or len(bias.shape) != 1:
            raise _err(ox.INVALID_SHAPE, "conv2d expects NCHW input, OIHW weight, and rank-1 bias")
        if stride == 0 or groups == 0:
            raise _err(ox.INVALID_SHAPE, "conv2d stride and groups must be non-zero")
        n, cin, h, w = self.shape
        cout, wc, kh, kw = weight.shape
        if kh == 0 or kw == 0 or kh != kw:
            raise _err(ox.INVALID_SHAPE, "conv2d currently requires a non-zero square kernel")
        if cin % groups or cout % groups or wc != cin // groups or bias.shape[0] != cout:
            raise _err(ox.INVALID_SHAPE, "conv2d group/channel dimensions are inconsistent")
        ph, pw = h + 2 * padding, w + 2 * padding
        if ph < kh or pw < kw:
            raise _err(ox.INVALID_SHAPE, "conv2d kernel exceeds input")
        out = (n, cout, (ph - kh) // stride + 1, (pw - kw) // stride + 1)
        return Tensor(out, "conv2d", (self, weight, bias), stride=int(stride),
                      padding=int(padding), groups=int(groups))

    # tensor/mod.rs:239-272
    def avg_pool2d(self, kernel, stride):
        if len(self.shape) != 4:
            raise _err(ox.INVALID_SHAPE, "avg_pool2d expects NCHW input")
        kernel, stride = tuple(int(k) for k in kernel), tuple(int(s) for s in stride)
        if 0 in kernel or 0 in stride:
            raise _err(ox.INVALID_SHAPE, "avg_pool2d kernel and stride must be non-zero")
        n, c, h, w = self.shape
        if kernel[0] > h or kernel[1] > w:
            raise _err(ox.INVALID_SHAPE, "avg_pool2d kernel exceeds input")
        out = (n, c, (h - kernel[0]) // stride[0] + 1, (w - kernel[1]) // stride[1] + 1)
        return Tensor(out, "avg_pool2d", (self,), kernel=kernel, stride=stride)

    def global_avg_pool2d(self):
        if len(self.shape) != 4:
            raise _err(ox.INVALID_SHAPE, "global_avg_pool2d expects NCHW input")
        return self.avg_pool2d(self.shape[2:], self.shape[2:])

    # tensor/mod.rs:331-389
    def batch_norm2d(self, weight, bias, state: BatchNormState, training: bool,
                     momentum: float, epsilon: float):
        if len(self.shape) != 4 or len(weight.shape) != 1 or len(bias.shape) != 1:
            raise _err(ox.INVALID_SHAPE, "batch_norm2d expects NCHW input and rank-1 weight/bias")
        c = self.shape[1]
        if weight.shape != (c,) or bias.shape != (c,):
            raise _err(ox.INVALID_SHAPE, "batch_norm2d weight/bias must match the channel count")
        m32, e32 = np.float32(momentum), np.float32(epsilon)
        if not np.isfinite(m32) or not 0.0 <= m32 <= 1.0:
            raise _err(ox.EXECUTION, "batch_norm2d momentum must be finite and in 0..=1")
        if not np.isfinite(e32) or e32 <= 0.0:
            raise _err(ox.EXECUTION, "batch_norm2d epsilon must be positive and finite")
        if state.channels != c:
            raise _err(ox.INVALID_SHAPE,
                       "batch_norm2d running statistics must match the channel count")
        return Tensor(self.shape, "batch_norm2d", (self, weight, bias), state=state,
                      training=bool(training), momentum=float(m32), epsilon=float(e32))

    # tensor/mod.rs:303-329
    def cross_entropy(self, targets):
        if len(self.shape) != 2 or len(targets.shape) != 1 or self.shape[0] != targets.shape[0]:
            raise _err(ox.INVALID_SHAPE,
                       "cross_entropy expects [batch, classes] logits and [batch] targets")
        return Tensor((1,), "cross_entropy", (self, targets))


def input(shape, requires_grad: bool = False) -> Tensor:  # noqa: A001 - Tensor::placeholder
    """A value fed per run (a placeholder, tensor/mod.rs:520-522; ``requires_grad`` gives it a
    gradient as a Data tensor has in the reference's autograd)."""
    shape = tuple(int(s) for s in shape)
    if not shape:
        raise _err(ox.INVALID_SHAPE, "scalar shapes are not implemented")
    return Tensor(shape, "input", requires_grad=bool(requires_grad))


def constant(values, shape=None) -> Tensor:
    arr = np.ascontiguousarray(values, dtype=np.float32)
    if shape is not None:
        arr = np.broadcast_to(arr, shape).astype(np.float32)
    if arr.ndim == 0:
        arr = arr.reshape(1)
    return Tensor(arr.shape, "constant", value=arr.ravel())


def parameter_tensor(param) -> Tensor:
    """The lazy leaf of an ``nn.Parameter`` (device values, trainable)."""
    return Tensor(param.shape, "parameter", param=param)


def postorder(outputs: Sequence[Tensor]) -> list[Tensor]:
    """Every node below ``outputs`` once, operands before their users, operands visited in
    order (the order a recursive lowering creates nodes in)."""
    order, seen = [], set()
    stack = [(t, False) for t in reversed(list(outputs))]
    while stack:
        t, expanded = stack.pop()
        if t.id in seen:
            continue
        if expanded:
            seen.add(t.id)
            order.append(t)
            continue
        stack.append((t, True))
        for a in reversed(t.args):
            if a.id not in seen:
                stack.append((a, False))
    return order


# ----------------------------------------------------------------------------- nets

class Net:
    """The traced graph in liboxide_hip (``oxh_net``): one node per distinct lazy node, in the
    lowering's creation order.  A parameter lowers once however many lazy leaves name it;
    constants are uploaded here and kept alive with the net."""

    def __init__(self, outputs: Sequence[Tensor]):
        import torch

        h = _vp()
        _call("oxh_net_create", ctypes.byref(h))
        self.handle = h.value
        self.node: dict[int, int] = {}
        self._params: dict[int, int] = {}
        self._keep = []
        dev = torch.device("cuda:0") if torch.cuda.is_available() else None
        for t in postorder(outputs):
            self.node[t.id] = self._lower(t, dev)

    def _shape(self, t):
        arr = (_u64 * len(t.shape))(*t.shape)
        return len(t.shape), arr

    def _lower(self, t: Tensor, dev) -> int:
        import torch

        out = _u32()
        n = lambda x: self.node[x.id]  # noqa: E731
        rank, shape = self._shape(t)
        h = self.handle
        if t.kind == "input":
            _call("oxh_net_input", h, rank, shape, int(t.requires_grad), ctypes.byref(out))
        elif t.kind == "parameter":
            p = t.attrs["param"]
            if id(p) in self._params:
                return self._params[id(p)]
            _call("oxh_net_parameter", h, rank, shape, p.data_ptr(), ctypes.byref(out))
            self._params[id(p)] = out.value
        elif t.kind == "constant":
            if dev is None:
                raise _err(ox.EXECUTION, "constants need a GPU to live on")
            values = torch.from_numpy(np.ascontiguousarray(t.value, np.float32)).to(dev)
            self._keep.append(values)
            _call("oxh_net_constant", h, rank, shape, values.data_ptr(), ctypes.byref(out))
        elif t.kind in ("add", "mul"):
            _call("oxh_net_" + t.kind, h, n(t.args[0]), n(t.args[1]), ctypes.byref(out))
        elif t.kind == "relu":
            _call("oxh_net_relu", h, n(t.args[0]), ctypes.byref(out))
        elif t.kind == "reshape":
            _call("oxh_net_reshape", h, n(t.args[0]), rank, shape, ctypes.byref(out))
        elif t.kind == "conv2d":
            a = t.attrs
            _call("oxh_net_conv2d", h, n(t.args[0]), n(t.args[1]), n(t.args[2]), a["stride"],
                  a["padding"], a["groups"], ctypes.byref(out))
        elif t.kind == "avg_pool2d":
            (kh, kw), (sh, sw) = t.attrs["kernel"], t.attrs["stride"]
            _call("oxh_net_avg_pool2d", h, n(t.args[0]), kh, kw, sh, sw, ctypes.byref(out))
        elif t.kind == "batch_norm2d":
            a = t.attrs
            st = a["state"]
            _call("oxh_net_batch_norm2d", h, n(t.args[0]), n(t.args[1]), n(t.args[2]),
                  st.running_mean.data_ptr(), st.running_variance.data_ptr(),
                  int(a["training"]), a["momentum"], a["epsilon"], ctypes.byref(out))
        elif t.kind == "cross_entropy":
            _call("oxh_net_cross_entropy", h, n(t.args[0]), n(t.args[1]), ctypes.byref(out))
        else:
            raise _err(ox.TRACE, f"no device kernel serves {t.kind} on this path")
        return out.value

    def node_shape(self, t: Tensor) -> tuple:
        rank, shape = _u32(), (_u64 * 4)()
        _call("oxh_net_node_shape", self.handle, self.node[t.id], ctypes.byref(rank), shape)
        return tuple(shape[:rank.value])

    def close(self):
        if getattr(self, "handle", None) and ox._lib is not None:
            ox.lib().oxh_net_destroy(self.handle)
            self.handle = None

    __del__ = close


class Program:
    """A device program built from a net (``oxh_net_forward_program`` /
    ``oxh_net_training_program``): ``feed`` the inputs, ``run`` (or ``capture`` once and
    ``replay``), then read ``value`` / ``gradient`` of any node; ``ops`` lists the launch
    groups."""

    def __init__(self, handle: int, net: Net):
        self.handle, self.net = handle, net
        stream = _vp()
        _call("oxh_program_stream", handle, ctypes.byref(stream))
        self.stream_handle = stream.value
        count = _u64()
        _call("oxh_program_op_count", handle, ctypes.byref(count))
        self.ops = [T.Op(handle, i, self.stream_handle) for i in range(count.value)]

    def torch_stream(self):
        import torch

        return torch.cuda.ExternalStream(self.stream_handle)

    def _node(self, t: Tensor) -> int:
        if t.kind == "parameter":
            return self.net._params[id(t.attrs["param"])]
        return self.net.node[t.id]

    def value(self, t: Tensor) -> T.DeviceView:
        ptr = _vp()
        _call("oxh_program_value", self.handle, self._node(t), ctypes.byref(ptr))
        return T.DeviceView(ptr.value, t.shape, stream=self.stream_handle)

    def gradient(self, t: Tensor):
        ptr = _vp()
        _call("oxh_program_gradient", self.handle, self._node(t), ctypes.byref(ptr))
        return None if not ptr.value else T.DeviceView(ptr.value, t.shape,
                                                        stream=self.stream_handle)

    def feed(self, t: Tensor, values) -> None:
        if t.kind != "input":
            raise _err(ox.TRACE, "only inputs are fed")
        self.value(t).copy_from(values)

    def run(self) -> None:
        _call("oxh_program_run", self.handle)

    def capture(self) -> None:
        _call("oxh_program_capture", self.handle)

    def replay(self) -> None:
        _call("oxh_program_replay", self.handle)

    def synchronize(self) -> None:
        ox.check(ox.lib().oxh_stream_synchronize(self.stream_handle))

    def check(self) -> None:
        """Waits; InvalidShape if a cross entropy met a target that is not a class index."""
        _call("oxh_program_check", self.handle)

    def steps(self) -> int:
        s = ctypes.c_int32()
        _call("oxh_program_steps", self.handle, ctypes.byref(s))
        return s.value

    def close(self) -> None:
        if getattr(self, "handle", None) and ox._lib is not None:
            ox.lib().oxh_program_destroy(self.handle)
            self.handle = None

    __del__ = close


def forward_program(output: Tensor, inputs: Sequence[Tensor] = ()) -> Program:
    """The eager device evaluation of ``output`` (runtime.rs:125-379); ``inputs`` are lowered
    first, in order, whether the output reads them or not."""
    net = Net(list(inputs) + [output])
    h = _vp()
    _call("oxh_net_forward_program", net.handle, net.node[output.id], ctypes.byref(h))
    return Program(h.value, net)


def training_program(loss: Tensor, adamw=None) -> Program:
    """Forward, reverse mode from the one-element ``loss`` (Tensor::backward), and with an
    ``nn.AdamW`` one optimizer step over every parameter the loss reaches."""
    net = Net([loss])
    h = _vp()
    cfg = None
    if adamw is not None:
        cfg = AdamWConfig(adamw.learning_rate, adamw.weight_decay, adamw.betas[0],
                          adamw.betas[1], adamw.epsilon)
    _call("oxh_net_training_program", net.handle, net.node[loss.id],
          ctypes.byref(cfg) if cfg is not None else None, ctypes.byref(h))
    return Program(h.value, net)
