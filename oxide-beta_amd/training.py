"""MobileNetV4-Conv-S (MNIST variant) and its training step: Python front end of the native
executor in liboxide_hip.so (``oxh_mnv4_*``, ``oxh_model_*``, ``oxh_trainer_*``,
``oxh_evaluator_*``, ``oxh_program_*``).

Mirrors the reference's model and driver -- MobileNetV4ConvSmall (mobilenet_v4.rs:84-321),
the step of examples/mnist_training.rs:75-92 (forward, cross entropy, backward, AdamW with
lr 1e-3 / weight decay 1e-4), model.eval() + count_correct for the test set, save / load_mnist
-- while the library traces the step once into a fixed launch list over device buffers
allocated at creation and replays it from one hipGraph.  Each launch group is open to
inspection (``Op``: kind, the tensors it reads / writes / updates with their roles, scalar
arguments) and can be launched alone, so a checker can recompute it independently.
"""

from __future__ import annotations

import ctypes

import numpy as np

import oxide_hip as ox

BN_MOMENTUM, BN_EPSILON = 0.1, 1e-5

_u64, _vp, _f32 = ctypes.c_uint64, ctypes.c_void_p, ctypes.c_float


class OpTensor(ctypes.Structure):
    _fields_ = [("role", ctypes.c_char_p), ("data", _vp), ("shape", _u64 * 4),
                ("rank", ctypes.c_uint32), ("access", ctypes.c_int), ("dtype", ctypes.c_int)]


class OpAttr(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("value", ctypes.c_double)]


class OpInfo(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_char_p), ("name", ctypes.c_char_p),
                ("tensor_count", ctypes.c_uint32), ("tensors", ctypes.POINTER(OpTensor)),
                ("attr_count", ctypes.c_uint32), ("attrs", ctypes.POINTER(OpAttr))]


_SIGNATURES = {
    "oxh_mnv4_create": [_u64, _u64, _u64, ctypes.POINTER(_vp)],
    "oxh_mnv4_describe": [_u64, _u64, _u64, _u64, ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                          ctypes.POINTER(_u64), _vp, _u64, ctypes.POINTER(_u64)],
    "oxh_model_destroy": [_vp],
    "oxh_model_info": [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                       ctypes.POINTER(ctypes.c_int)],
    "oxh_model_parameter": [_vp, _u64, ctypes.POINTER(_u64), _u64 * 4, ctypes.POINTER(_vp)],
    "oxh_model_batch_norm": [_vp, _u64, ctypes.POINTER(_u64), ctypes.POINTER(_vp),
                             ctypes.POINTER(_vp)],
    "oxh_model_set_training": [_vp, ctypes.c_int],
    "oxh_model_save": [_vp, ctypes.c_char_p],
    "oxh_model_load_mnist": [ctypes.c_char_p, ctypes.POINTER(_vp)],
    "oxh_trainer_create": [_vp, _u64, _f32, _f32, ctypes.POINTER(_vp)],
    "oxh_trainer_destroy": [_vp],
    "oxh_trainer_buffers": [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                            ctypes.POINTER(_vp)],
    "oxh_trainer_program": [_vp, ctypes.POINTER(_vp)],
    "oxh_trainer_loss": [_vp, ctypes.POINTER(_f32)],
    "oxh_trainer_steps": [_vp, ctypes.POINTER(ctypes.c_int32)],
    "oxh_evaluator_create": [_vp, _u64, ctypes.POINTER(_vp)],
    "oxh_evaluator_destroy": [_vp],
    "oxh_evaluator_buffers": [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    "oxh_evaluator_program": [_vp, ctypes.POINTER(_vp)],
    "oxh_evaluator_predict": [_vp],
    "oxh_program_stream": [_vp, ctypes.POINTER(_vp)],
    "oxh_program_run": [_vp],
    "oxh_program_capture": [_vp],
    "oxh_program_replay": [_vp],
    "oxh_program_op_count": [_vp, ctypes.POINTER(_u64)],
    "oxh_program_op": [_vp, _u64, ctypes.POINTER(OpInfo)],
    "oxh_program_run_op": [_vp, _u64],
}

_bound = None


def _lib():
    """The library with this module's entry points typed (once)."""
    global _bound
    if _bound is None:
        handle = ox.lib()
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


# ----------------------------------------------------------------------------- device views

class DeviceView:
    """A device buffer owned by the library (fp32 or int32), with host copies on demand."""

    def __init__(self, ptr: int, shape, dtype=np.float32, stream: int | None = None):
        self.ptr, self.shape = int(ptr), tuple(int(d) for d in shape)
        self.dtype, self.stream = np.dtype(dtype), stream

    def numel(self) -> int:
        return int(np.prod(self.shape))

    def data_ptr(self) -> int:
        return self.ptr

    def host(self) -> np.ndarray:
        """Waits for all device work, then copies the buffer to the host."""
        import torch

        torch.cuda.synchronize()
        out = np.empty(self.shape, self.dtype)
        if out.size:
            ox.check(ox.lib().oxh_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, self.stream))
        return out

    def copy_from(self, values) -> None:
        import torch

        values = np.ascontiguousarray(values, self.dtype).reshape(self.shape)
        torch.cuda.synchronize()
        ox.check(ox.lib().oxh_memcpy_h2d_async(self.ptr, values.ctypes.data, values.nbytes,
                                               self.stream))
        ox.check(ox.lib().oxh_stream_synchronize(self.stream))

    def view(self, shape) -> "DeviceView":
        if int(np.prod(shape)) != self.numel():
            raise ox.OxideError(ox.INVALID_SHAPE, "view must keep the element count")
        return DeviceView(self.ptr, shape, self.dtype, self.stream)

    def __repr__(self):
        return f"DeviceView(0x{self.ptr:x}, {self.shape}, {self.dtype})"


class Op:
    """One launch group of a program (oxh_program_op): ``kind``, ``name``; ``reads`` /
    ``writes`` map unique roles to views; ``inplace`` lists the views it updates in place
    (their values before the launch are part of its input); ``by_role`` maps every role to
    its views in order; ``attrs`` holds the scalar arguments; ``accumulate_into`` is set when
    the group adds its ``contribution`` into an existing gradient, and ``side_accumulate`` maps
    a written role (a parameter gradient of a value with several consumers) to the gradient it
    is added into after the launch."""

    def __init__(self, program, index: int, stream: int):
        info = OpInfo()
        _call("oxh_program_op", program, index, ctypes.byref(info))
        self._program, self.index = program, index
        self.kind, self.name = info.kind.decode(), info.name.decode()
        self.reads, self.writes, self.inplace, self.by_role = {}, {}, [], {}
        self.accumulate_into = None
        self.side_accumulate = {}
        for i in range(info.tensor_count):
            t = info.tensors[i]
            role = t.role.decode()
            v = DeviceView(t.data, tuple(t.shape[:t.rank]),
                           np.int32 if t.dtype == 1 else np.float32, stream)
            self.by_role.setdefault(role, []).append(v)
            if role == "accumulate_into":
                self.accumulate_into = v
                self.inplace.append(v)
            elif role.startswith("accumulate_into:"):
                self.side_accumulate[role.split(":", 1)[1]] = v
                self.inplace.append(v)
            elif t.access == 0:
                self.reads.setdefault(role, v)
            elif t.access == 1:
                self.writes.setdefault(role, v)
            else:
                self.inplace.append(v)
        self.attrs = {info.attrs[i].name.decode(): info.attrs[i].value
                      for i in range(info.attr_count)}
        for k in ("stride", "padding", "groups"):
            if k in self.attrs:
                self.attrs[k] = int(self.attrs[k])
        if "kernel_h" in self.attrs:
            self.attrs["kernel"] = (int(self.attrs["kernel_h"]), int(self.attrs["kernel_w"]))
            self.attrs["stride"] = (int(self.attrs["stride_h"]), int(self.attrs["stride_w"]))
        if self.kind == "adamw":
            r = self.by_role
            self.attrs["tensors"] = list(zip(r["parameter"], r["gradient"], r["first_moment"],
                                             r["second_moment"]))
            self.attrs["step_counter"] = r["step"][0]
        for role in ("running_mean", "running_variance", "pre_running_mean",
                     "pre_running_variance"):
            if role in self.by_role and self.kind != "batch_norm2d_eval_forward":
                self.attrs[role] = self.by_role[role][0]

    def launch(self) -> None:
        _call("oxh_program_run_op", self._program, self.index)


class _Program:
    def __init__(self, handle: int):
        self.handle = handle
        stream = _vp()
        _call("oxh_program_stream", handle, ctypes.byref(stream))
        self.stream_handle = stream.value
        count = _u64()
        _call("oxh_program_op_count", handle, ctypes.byref(count))
        self.ops = [Op(handle, i, self.stream_handle) for i in range(count.value)]

    def torch_stream(self):
        import torch

        return torch.cuda.ExternalStream(self.stream_handle)


# ----------------------------------------------------------------------------- model

class Parameter:
    def __init__(self, shape, value: DeviceView):
        self.shape, self.value = tuple(shape), value


class BatchNorm2d:
    def __init__(self, channels, running_mean: DeviceView, running_variance: DeviceView):
        self.channels = channels
        self.device_running_mean, self.device_running_variance = running_mean, running_variance


class MobileNetV4ConvSmall:
    """mobilenet_v4.rs:84-321 with its parameters and BatchNorm state on the device
    (oxh_mnv4_create); ``mnist()`` maps [N, 1, 28, 28] to 10 logits."""

    def __init__(self, num_classes=10, input_channels=1, input_resolution=28, _handle=None):
        if _handle is None:
            h = _vp()
            _call("oxh_mnv4_create", num_classes, input_channels, input_resolution,
                  ctypes.byref(h))
            _handle = h.value
        self._handle = _handle
        self.num_classes, self.input_channels = num_classes, input_channels
        self.input_resolution = input_resolution

    @classmethod
    def mnist(cls):
        return cls(10, 1, 28)

    @classmethod
    def new(cls, num_classes):
        """The 224 x 224 RGB network of supplement table 11."""
        return cls(num_classes, 3, 224)

    @classmethod
    def load_mnist(cls, path) -> "MobileNetV4ConvSmall":
        """load_mnist (mobilenet_v4.rs:266-321), in inference mode."""
        h = _vp()
        _call("oxh_model_load_mnist", str(path).encode(), ctypes.byref(h))
        return cls(10, 1, 28, _handle=h.value)

    @staticmethod
    def describe(num_classes=10, input_channels=1, input_resolution=28, batch=1) -> dict:
        """Host-only: parameter tensors / values, BatchNorm layers and every block's output
        shape (forward_with_shapes, mobilenet_v4.rs:182-195)."""
        p, v, b, n = _u64(), _u64(), _u64(), _u64()
        shapes = (_u64 * (4 * 64))()
        _call("oxh_mnv4_describe", num_classes, input_channels, input_resolution, batch,
              ctypes.byref(p), ctypes.byref(v), ctypes.byref(b), shapes, 64, ctypes.byref(n))
        blocks = [tuple(shapes[i * 4:i * 4 + 4]) for i in range(n.value)]
        blocks[-1] = blocks[-1][:2]  # the reshaped logits [N, classes]
        return {"parameters": p.value, "values": v.value, "batch_norms": b.value,
                "block_shapes": blocks}

    def _info(self):
        p, b, v, t = _u64(), _u64(), _u64(), ctypes.c_int()
        _call("oxh_model_info", self._handle, ctypes.byref(p), ctypes.byref(b), ctypes.byref(v),
              ctypes.byref(t))
        return p.value, b.value, v.value, bool(t.value)

    @property
    def training(self) -> bool:
        return self._info()[3]

    def train(self):
        _call("oxh_model_set_training", self._handle, 1)

    def eval(self):
        _call("oxh_model_set_training", self._handle, 0)

    def parameter_count(self) -> int:
        return self._info()[2]

    def parameters(self) -> list:
        """Visit order: per conv weight, bias; per BatchNorm gamma, beta."""
        out = []
        for i in range(self._info()[0]):
            rank, shape, ptr = _u64(), (_u64 * 4)(), _vp()
            _call("oxh_model_parameter", self._handle, i, ctypes.byref(rank), shape,
                  ctypes.byref(ptr))
            dims = tuple(shape[:rank.value])
            out.append(Parameter(dims, DeviceView(ptr.value, dims)))
        return out

    def batch_norms(self) -> list:
        out = []
        for i in range(self._info()[1]):
            c, rm, rv = _u64(), _vp(), _vp()
            _call("oxh_model_batch_norm", self._handle, i, ctypes.byref(c), ctypes.byref(rm),
                  ctypes.byref(rv))
            out.append(BatchNorm2d(c.value, DeviceView(rm.value, (c.value,)),
                                   DeviceView(rv.value, (c.value,))))
        return out

    def save(self, path) -> None:
        """OXTR checkpoint of the current device state (mobilenet_v4.rs:217-264)."""
        _call("oxh_model_save", self._handle, str(path).encode())

    def __del__(self):
        if getattr(self, "_handle", None) and ox._lib is not None:
            _lib().oxh_model_destroy(self._handle)
            self._handle = None


# ----------------------------------------------------------------------------- step

class TrainingStep:
    """examples/mnist_training.rs:75-92 on the device (oxh_trainer_*): ``set_batch`` (or a
    device gather into ``input`` / ``targets``), then ``run_eager()`` or ``capture()`` once and
    ``replay()`` per step; ``loss_value()`` reads the loss."""

    def __init__(self, model: MobileNetV4ConvSmall, batch: int, learning_rate=1e-3,
                 weight_decay=1e-4):
        import torch

        h = _vp()
        _call("oxh_trainer_create", model._handle, batch, learning_rate, weight_decay,
              ctypes.byref(h))
        self._handle, self.model, self.batch = h.value, model, batch
        self.hyper = dict(learning_rate=learning_rate, weight_decay=weight_decay, beta1=0.9,
                          beta2=0.999, epsilon=1e-8)
        prog = _vp()
        _call("oxh_trainer_program", self._handle, ctypes.byref(prog))
        self._program = _Program(prog.value)
        self.ops = self._program.ops
        s = self._program.stream_handle
        img, lbl, lg, loss = _vp(), _vp(), _vp(), _vp()
        _call("oxh_trainer_buffers", self._handle, ctypes.byref(img), ctypes.byref(lbl),
              ctypes.byref(lg), ctypes.byref(loss))
        r = model.input_resolution
        self.input = DeviceView(img.value, (batch, model.input_channels, r, r), stream=s)
        self.targets = DeviceView(lbl.value, (batch,), stream=s)
        self.logits = DeviceView(lg.value, (batch, model.num_classes), stream=s)
        self.loss = DeviceView(loss.value, (1,), stream=s)
        self.stream = self._program.torch_stream()
        self.params = model.parameters()
        self._classes = torch.empty(batch, dtype=torch.int32, device="cuda")

    def set_batch(self, images: np.ndarray, labels: np.ndarray) -> None:
        """Uploads one batch: images [N, C, H, W] float32, labels [N] class indices."""
        self.input.copy_from(images)
        self.targets.copy_from(labels)

    def run_eager(self, before=None, after=None) -> None:
        """Launches the step group by group; ``before`` / ``after`` run around each ``Op``."""
        if before is None and after is None:
            _call("oxh_program_run", self._program.handle)
            return
        for op in self.ops:
            if before is not None:
                before(op)
            op.launch()
            if after is not None:
                after(op)

    def capture(self) -> None:
        _call("oxh_program_capture", self._program.handle)

    def replay(self) -> None:
        _call("oxh_program_replay", self._program.handle)

    def synchronize(self) -> None:
        self.stream.synchronize()

    def loss_value(self) -> float:
        """The last step's loss; InvalidShape if a label was not a class index."""
        v = _f32()
        _call("oxh_trainer_loss", self._handle, ctypes.byref(v))
        return v.value

    def predicted_classes(self) -> np.ndarray:
        """argmax of each row of the last logits (ties go to the last index)."""
        import torch

        self.synchronize()
        ox.check(ox.lib().oxh_argmax_rows(self._program.stream_handle, self.batch,
                                          self.model.num_classes, self.logits.ptr,
                                          self._classes.data_ptr()))
        self.synchronize()
        torch.cuda.synchronize()
        return self._classes.cpu().numpy().astype(np.int64)

    def steps_taken(self) -> int:
        v = ctypes.c_int32()
        _call("oxh_trainer_steps", self._handle, ctypes.byref(v))
        return v.value

    def sync_to_model(self) -> None:
        """Waits for the step; the model's parameters and running statistics are the device
        buffers this trainer updates (``save`` copies them to the host itself)."""
        self.synchronize()

    def __del__(self):
        if getattr(self, "_handle", None) and ox._lib is not None:
            _lib().oxh_trainer_destroy(self._handle)
            self._handle = None


class EvalForward:
    """The inference-mode forward (BatchNorm from the running statistics,
    evaluation.rs:448-488,560-575) of ``batch`` images with argmax predictions, as
    mnist_training.rs evaluates the test set (oxh_evaluator_*).  It reads the model's
    current device parameters, so it sees every step of a trainer over the same model."""

    def __init__(self, model: MobileNetV4ConvSmall, batch: int, source=None):
        if source is not None and source.model is not model:
            raise ox.OxideError(ox.INVALID_SHAPE, "source trains another model")
        h = _vp()
        _call("oxh_evaluator_create", model._handle, batch, ctypes.byref(h))
        self._handle, self.model, self.batch = h.value, model, batch
        prog = _vp()
        _call("oxh_evaluator_program", self._handle, ctypes.byref(prog))
        self._program = _Program(prog.value)
        self.ops = self._program.ops
        s = self._program.stream_handle
        img, lg, pred = _vp(), _vp(), _vp()
        _call("oxh_evaluator_buffers", self._handle, ctypes.byref(img), ctypes.byref(lg),
              ctypes.byref(pred))
        r = model.input_resolution
        self.input = DeviceView(img.value, (batch, model.input_channels, r, r), stream=s)
        self.logits = DeviceView(lg.value, (batch, model.num_classes), stream=s)
        self.predictions = DeviceView(pred.value, (batch,), np.int32, stream=s)
        self.stream = self._program.torch_stream()

    def set_images(self, images: np.ndarray) -> None:
        self.input.copy_from(images)

    def run(self, before=None, after=None) -> None:
        if before is None and after is None:
            _call("oxh_program_run", self._program.handle)
            return
        for op in self.ops:
            if before is not None:
                before(op)
            op.launch()
            if after is not None:
                after(op)

    def capture(self) -> None:
        _call("oxh_program_capture", self._program.handle)

    def replay(self) -> None:
        _call("oxh_program_replay", self._program.handle)

    def predicted_classes(self) -> np.ndarray:
        _call("oxh_evaluator_predict", self._handle)
        return self.predictions.host().astype(np.int64)

    def __del__(self):
        if getattr(self, "_handle", None) and ox._lib is not None:
            _lib().oxh_evaluator_destroy(self._handle)
            self._handle = None


def op_bytes(op: Op) -> tuple[str, int]:
    """(category, algorithmic HBM bytes) of one launch group: every tensor it must read or
    write, once (fp32).  Categories: the hot-path kernel families (batch_norm2d, elementwise,
    cross_entropy, adamw) and the layers around them (conv2d, avg_pool2d)."""
    nb = lambda t: t.numel() * 4  # noqa: E731
    acc = 3 * nb(op.accumulate_into) if op.accumulate_into is not None else 0
    k = op.kind
    if k in ("batch_norm2d_forward", "batch_norm2d_relu_forward"):
        return "batch_norm2d", 2 * nb(op.reads["x"])                       # x in, y out
    if k == "batch_norm2d_add_forward":
        return "batch_norm2d", 3 * nb(op.reads["x"])                       # x, shortcut in; y out
    if k == "batch_norm2d_backward":
        return "batch_norm2d", 3 * nb(op.reads["x"]) + acc                 # g, x in; dx out
    if k == "batch_norm2d_relu_backward":
        return "batch_norm2d", 4 * nb(op.reads["x"]) + acc                 # g, y, x in; dx out
    if k.startswith("batch_norm2d") and "depthwise" in k and k.endswith("forward"):
        # BN input (and residual) in; its output, the convolution output and the layer output
        return ("batch_norm2d+conv2d+batch_norm2d",
                (2 + ("pre_residual" in op.reads)) * nb(op.reads["pre_x"]) +
                2 * nb(op.writes["y"]))
    if k.startswith("batch_norm2d") and "depthwise" in k:
        # g (, y), convolution output, its input and the BN input in; output gradients out
        outs = nb(op.reads["gradient"]) * (3 + ("y" in op.reads))
        return "batch_norm2d+conv2d+batch_norm2d", outs + 3 * nb(op.reads["x"]) + acc
    if k.startswith("depthwise_conv2d_batch_norm") and k.endswith("forward"):
        # x in; convolution output and layer output out
        return "conv2d+batch_norm2d", nb(op.reads["x"]) + 2 * nb(op.writes["y"])
    if k.startswith("depthwise_conv2d_batch_norm"):
        # g (, y), convolution output, x (, addend) in; output and input gradients out
        outs = nb(op.reads["gradient"]) * (3 + ("y" in op.reads))
        ins = nb(op.reads["x"]) * (1 + ("contribution" in op.writes) + ("addend" in op.reads))
        return "conv2d+batch_norm2d", outs + ins + acc
    if k == "add_forward":
        return "elementwise", 3 * nb(op.reads["a"])
    if k == "relu_forward":
        return "elementwise", 2 * nb(op.reads["x"])
    if k == "relu_backward":
        return "elementwise", 3 * nb(op.reads["gradient"]) + acc           # g, x in; out
    if k == "add_backward":
        return "elementwise", 2 * nb(op.reads["gradient"]) + acc           # copy of g
    if k == "cross_entropy":
        return "cross_entropy", 2 * nb(op.reads["logits"])
    if k == "adamw":
        return "adamw", sum(7 * nb(t[0]) for t in op.attrs["tensors"])
    if k.startswith("avg_pool2d"):
        return "avg_pool2d", 0
    return "conv2d", 0
