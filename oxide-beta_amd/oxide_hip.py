"""Python front end of liboxide_hip.so (the MI355X backend of oxide-torch's tensor hot path).

The C ABI (include/oxide_hip.h) is the product boundary; this module binds it with ctypes and
mirrors the reference's backend surface on this path so tests and benchmarks read like the
reference's own code:

* ``LoadedModule``: the kernel launchers of ``oxide_torch_cuda::load_kernels``
  (crates/oxide-torch-cuda/src/lib.rs:19-30, launchers from kernel_module.rs) -- ``add``,
  ``mul``, ``relu``, ``mul_backward``, ``relu_backward``, ``accumulate``,
  ``batch_norm_statistics``, ``batch_norm_update_running``, ``batch_norm_running_inverse_std``,
  ``batch_norm_apply``, ``batch_norm_affine_backward``, ``batch_norm_input_backward``,
  ``cross_entropy_forward``, ``cross_entropy_backward``, ``adamw`` -- plus the fused entry
  points.  Arguments are device tensors (torch is only the allocator and stream provider).
* ``HipGraphExec``: ``CudaGraphExec::{capture, launch}`` (cuda_graph.rs:47-165).

The lazy graph, its device programs and autograd are in tensor.py, the modules in nn.py, the
JIT (fused plans and their eager fallback) in jit.py.

Errors raise ``OxideError`` whose ``kind`` names the reference's Error variant
(crates/oxide-torch/src/error.rs): ``InvalidShape``, ``Execution``, ``Hip`` (for ``Cuda``),
``Trace``.  There is no CPU fallback: if the library is missing every call fails.
"""

from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path
from typing import Callable

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "liboxide_hip.so"
HEADER_PATH = _HERE.parent / "include" / "oxide_hip.h"

OK, INVALID_SHAPE, EXECUTION, HIP_ERROR, TRACE = 0, 1, 2, 3, 4
_KINDS = {INVALID_SHAPE: "InvalidShape", EXECUTION: "Execution", HIP_ERROR: "Hip",
          TRACE: "Trace"}

PLAN_ADD, PLAN_MUL, PLAN_RELU = 1, 2, 3
PLAN_RELU_BACKWARD, PLAN_MUL_BACKWARD, PLAN_ACCUMULATE = 4, 5, 6


class OxideError(RuntimeError):
    """A failed C-ABI call; ``kind`` is the reference Error variant it maps to."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = _KINDS.get(status, f"status {status}")
        super().__init__(f"{self.kind}: {message}")


_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int32
_int = ctypes.c_int
_f32 = ctypes.c_float
_st = ctypes.c_int


class AdamWTensor(ctypes.Structure):
    _fields_ = [("parameter", _vp), ("gradient", _vp), ("first_moment", _vp),
                ("second_moment", _vp), ("n", _u64)]


class Conv2dShape(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint64) for f in (
        "batch", "in_channels", "height", "width", "out_channels", "kernel_h", "kernel_w",
        "stride", "padding", "groups")]


class Pool2dShape(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint64) for f in (
        "batch", "channels", "height", "width", "kernel_h", "kernel_w", "stride_h", "stride_w")]


class CheckpointTensor(ctypes.Structure):
    _fields_ = [("rank", ctypes.c_uint64), ("shape", ctypes.POINTER(ctypes.c_uint64)),
                ("len", ctypes.c_uint64), ("data", ctypes.POINTER(ctypes.c_float))]


_CS = ctypes.POINTER(Conv2dShape)
_PS = ctypes.POINTER(Pool2dShape)

_SIGNATURES = {
    "oxh_last_error": (ctypes.c_char_p, []),
    "oxh_version": (ctypes.c_char_p, []),
    "oxh_init": (_st, [_int]),
    "oxh_device_count": (_st, [ctypes.POINTER(_int)]),
    "oxh_stream_create": (_st, [ctypes.POINTER(_vp)]),
    "oxh_stream_destroy": (_st, [_vp]),
    "oxh_stream_synchronize": (_st, [_vp]),
    "oxh_alloc": (_st, [ctypes.POINTER(_vp), _u64]),
    "oxh_free": (_st, [_vp]),
    "oxh_memset0_async": (_st, [_vp, _u64, _vp]),
    "oxh_memcpy_h2d_async": (_st, [_vp, _vp, _u64, _vp]),
    "oxh_memcpy_d2h": (_st, [_vp, _vp, _u64, _vp]),
    "oxh_memcpy_d2d_async": (_st, [_vp, _vp, _u64, _vp]),
    "oxh_event_create": (_st, [ctypes.POINTER(_vp)]),
    "oxh_event_destroy": (_st, [_vp]),
    "oxh_event_elapsed_ms": (_st, [_vp, _vp, ctypes.POINTER(_f32)]),
    "oxh_time_next_launch": (_st, [_vp, _vp]),
    "oxh_add": (_st, [_vp, _vp, _vp, _vp, _u64]),
    "oxh_mul": (_st, [_vp, _vp, _vp, _vp, _u64]),
    "oxh_relu": (_st, [_vp, _vp, _vp, _u64]),
    "oxh_mul_backward": (_st, [_vp, _vp, _vp, _vp, _u64]),
    "oxh_relu_backward": (_st, [_vp, _vp, _vp, _vp, _u64]),
    "oxh_accumulate": (_st, [_vp, _vp, _vp, _vp, _u64]),
    "oxh_elementwise_chain_forward": (_st, [_vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_elementwise_chain_backward": (_st, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_workspace_size": (_st, [_u64, _u64, _u64, ctypes.POINTER(_u64)]),
    "oxh_batch_norm_statistics": (_st, [_vp, _u64, _u64, _u64, _f32, _vp, _vp, _vp, _vp, _vp,
                                        _u64]),
    "oxh_batch_norm_update_running": (_st, [_vp, _u64, _f32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oxh_batch_norm_running_inverse_std": (_st, [_vp, _u64, _f32, _vp, _vp]),
    "oxh_batch_norm_apply": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oxh_batch_norm_affine_backward": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _u64]),
    "oxh_batch_norm_input_backward": (_st, [_vp, _u64, _u64, _u64, _int, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp]),
    "oxh_batch_norm_forward_reduce": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _u64]),
    "oxh_batch_norm_forward_apply": (_st, [_vp, _u64, _u64, _u64, _f32, _f32, _vp, _vp, _vp,
                                           _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_backward_reduce": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp,
                                             _u64]),
    "oxh_batch_norm_backward_input": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_forward_train": (_st, [_vp, _u64, _u64, _u64, _f32, _f32, _vp, _vp, _vp,
                                           _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_forward_train_no_alloc": (_st, [_vp, _u64, _u64, _u64, _f32, _f32, _vp,
                                                    _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oxh_batch_norm_backward_train": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_relu_forward_train": (_st, [_vp, _u64, _u64, _u64, _f32, _f32, _vp, _vp,
                                                _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_relu_backward_train": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp,
                                                 _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_batch_norm_add_forward_train": (_st, [_vp, _u64, _u64, _u64, _f32, _f32, _vp, _vp, _vp,
                                               _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_conv_batch_norm_backward_train": (_st, [_vp, _u64, _u64, _u64, _vp, _vp, _vp, _vp, _vp,
                                                 _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_cross_entropy_workspace_size": (_st, [_u64, _u64, ctypes.POINTER(_u64)]),
    "oxh_cross_entropy_forward": (_st, [_vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_cross_entropy_backward": (_st, [_vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp]),
    "oxh_cross_entropy_forward_backward": (_st, [_vp, _u64, _u64, _vp, _vp, _vp, _vp, _vp, _vp,
                                                 _vp, _u64]),
    "oxh_adamw": (_st, [_vp, _f32, _f32, _f32, _f32, _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp,
                        _vp, _vp, _u64]),
    "oxh_adamw_corrections": (_st, [_f32, _f32, _i32, ctypes.POINTER(_f32),
                                    ctypes.POINTER(_f32)]),
    "oxh_adamw_multi_tensor": (_st, [_vp, _f32, _f32, _f32, _f32, _f32, _f32, _f32,
                                     ctypes.POINTER(AdamWTensor), _u32]),
    "oxh_adamw_table_layout": (_st, [ctypes.POINTER(AdamWTensor), _u32, ctypes.POINTER(_u32),
                                     ctypes.POINTER(_u64)]),
    "oxh_adamw_multi_tensor_table_step": (_st, [_vp, _f32, _f32, _f32, _f32, _f32, _vp, _vp,
                                                _vp, _u32, _u64]),
    "oxh_adamw_multi_tensor_step": (_st, [_vp, _f32, _f32, _f32, _f32, _f32, _vp,
                                          ctypes.POINTER(AdamWTensor), _u32]),
    "oxh_conv2d_output_size": (_st, [_CS, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "oxh_conv2d_forward": (_st, [_vp, _CS, _vp, _vp, _vp, _vp]),
    "oxh_conv2d_forward_serial": (_int, [_CS]),
    "oxh_conv2d_input_backward_serial": (_int, [_CS]),
    "oxh_conv2d_input_backward": (_st, [_vp, _CS, _vp, _vp, _vp]),
    "oxh_conv2d_input_backward_accumulate": (_st, [_vp, _CS, _vp, _vp, _vp, _vp]),
    "oxh_conv2d_weight_backward_workspace_size": (_st, [_CS, ctypes.POINTER(_u64)]),
    "oxh_conv2d_weight_backward": (_st, [_vp, _CS, _vp, _vp, _vp, _vp, _u64]),
    "oxh_conv2d_backward": (_st, [_vp, _CS, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u64]),
    "oxh_conv2d_bias_backward": (_st, [_vp, _CS, _vp, _vp, _vp, _u64]),
    "oxh_depthwise_conv_batch_norm_supported": (_int, [_CS]),
    "oxh_depthwise_conv_batch_norm_forward_train": (_st, [_vp, _CS, _int, _f32, _f32, _vp, _vp,
                                                          _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                          _vp, _vp]),
    "oxh_depthwise_conv_batch_norm_backward_train": (_st, [_vp, _CS, _vp, _vp, _vp, _vp, _vp,
                                                           _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                           _vp, _vp, _vp]),
    "oxh_batch_norm_depthwise_conv_batch_norm_supported": (_int, [_CS]),
    "oxh_batch_norm_depthwise_conv_batch_norm_forward_train": (
        _st, [_vp, _CS, _int, _f32, _f32] + [_vp] * 9 + [_int, _f32, _f32] + [_vp] * 10),
    "oxh_batch_norm_depthwise_conv_batch_norm_backward_train": (
        _st, [_vp, _CS] + [_vp] * 9 + [_int] + [_vp] * 14),
    "oxh_avg_pool2d_forward": (_st, [_vp, _PS, _vp, _vp]),
    "oxh_avg_pool2d_backward": (_st, [_vp, _PS, _vp, _vp]),
    "oxh_initialized_weights": (_st, [ctypes.POINTER(_u64), _u64, ctypes.POINTER(_f32)]),
    "oxh_argmax_rows": (_st, [_vp, _u64, _u64, _vp, _vp]),
    "oxh_checkpoint_save": (_st, [ctypes.c_char_p, ctypes.POINTER(CheckpointTensor), _u64]),
    "oxh_checkpoint_load": (_st, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "oxh_checkpoint_count": (_st, [_vp, ctypes.POINTER(_u64)]),
    "oxh_checkpoint_entry": (_st, [_vp, _u64, ctypes.POINTER(_u64),
                                   ctypes.POINTER(ctypes.POINTER(_u64)), ctypes.POINTER(_u64),
                                   ctypes.POINTER(ctypes.POINTER(_f32))]),
    "oxh_checkpoint_free": (_st, [_vp]),
    "oxh_idx_parse_images": (_st, [_vp, _u64, ctypes.POINTER(_u64)]),
    "oxh_idx_parse_labels": (_st, [_vp, _u64, ctypes.POINTER(_u64)]),
    "oxh_mnist_load": (_st, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "oxh_mnist_free": (_st, [_vp]),
    "oxh_mnist_split": (_st, [_vp, ctypes.c_int, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                              ctypes.POINTER(_u64)]),
    "oxh_mnist_batch_order": (_st, [_u64, ctypes.c_int, _vp]),
    "oxh_mnist_batch_host": (_st, [_vp, _vp, _u64, _vp, _u64, _vp, _vp]),
    "oxh_mnist_gather_batch": (_st, [_vp, _vp, _vp, _u64, _vp, _u64, _vp, _vp]),
    "oxh_graph_begin": (_st, [_vp]),
    "oxh_graph_end": (_st, [_vp, ctypes.POINTER(_vp)]),
    "oxh_graph_abort": (_st, [_vp]),
    "oxh_graph_launch": (_st, [_vp, _vp]),
    "oxh_graph_destroy": (_st, [_vp]),
    "oxh_plan_create": (_st, [_int, ctypes.POINTER(_vp)]),
    "oxh_plan_add_input": (_st, [_vp, _u64, ctypes.POINTER(_u32)]),
    "oxh_plan_add_constant": (_st, [_vp, _vp, _u64, ctypes.POINTER(_u32)]),
    "oxh_plan_add_workspace": (_st, [_vp, _u64, ctypes.POINTER(_u32)]),
    "oxh_plan_add_operation": (_st, [_vp, _u32, ctypes.POINTER(_u32), _u32, _u32]),
    "oxh_plan_set_output": (_st, [_vp, _u32]),
    "oxh_plan_compile": (_st, [_vp]),
    "oxh_plan_run": (_st, [_vp, ctypes.POINTER(_vp), _u32, _vp, _u64]),
    "oxh_plan_replay": (_st, [_vp]),
    "oxh_plan_launch": (_st, [_vp]),
    "oxh_plan_stream": (_st, [_vp, ctypes.POINTER(_vp)]),
    "oxh_plan_buffer": (_st, [_vp, _u32, ctypes.POINTER(_vp), ctypes.POINTER(_u64)]),
    "oxh_plan_destroy": (_st, [_vp]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads liboxide_hip.so (built by ``__graft_entry__.build()`` / ``make``)."""
    global _lib
    if _lib is None:
        # Tensors and streams handed to the C ABI come from torch, so the library must bind to
        # the HIP runtime torch loaded (same SONAME): import torch first.  Loading the library
        # first would bring in a second HIP runtime that torch then fails to initialise.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not LIB_PATH.exists():
            raise OxideError(HIP_ERROR, f"{LIB_PATH} is not built; run __graft_entry__.build()")
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def header_symbols() -> list[str]:
    """Every function the C ABI header declares."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(oxh_[a-z0-9_]+)\s*\(", text)))


def check(status: int) -> None:
    if status != OK:
        raise OxideError(status, lib().oxh_last_error().decode())


# ----------------------------------------------------------------------------- plumbing

def _ptr(t) -> int | None:
    """Device address of a torch tensor (or an int address, or None)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_contiguous():
        raise OxideError(INVALID_SHAPE, "tensors must be contiguous")
    return t.data_ptr()


def _f32_tensor(t, name: str):
    import torch

    if t.dtype != torch.float32 or not t.is_cuda:
        raise OxideError(INVALID_SHAPE, f"{name} must be a float32 device tensor")
    return t


def current_stream() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream


def _stream(stream) -> int | None:
    if stream is None:
        return current_stream()
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


class Workspace:
    """Device scratch for the reductions' partial sums, grown on demand."""

    def __init__(self):
        self._buf = None

    def get(self, nbytes: int):
        import torch

        if self._buf is None or self._buf.numel() < nbytes:
            # allocated on torch's stream; kernels may run on another stream
            torch.cuda.synchronize()
            self._buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
        return self._buf

    def ptr_bytes(self, nbytes: int) -> tuple[int, int]:
        b = self.get(nbytes)
        return b.data_ptr(), b.numel()


def batch_norm_workspace_size(batch: int, channels: int, spatial: int) -> int:
    out = _u64()
    check(lib().oxh_batch_norm_workspace_size(batch, channels, spatial, ctypes.byref(out)))
    return out.value


def cross_entropy_workspace_size(batch: int, classes: int) -> int:
    out = _u64()
    check(lib().oxh_cross_entropy_workspace_size(batch, classes, ctypes.byref(out)))
    return out.value


def adamw_corrections(beta1: float, beta2: float, step: int) -> tuple[float, float]:
    c1, c2 = _f32(), _f32()
    check(lib().oxh_adamw_corrections(beta1, beta2, step, ctypes.byref(c1), ctypes.byref(c2)))
    return c1.value, c2.value


class KernelTimer:
    """Start / stop events around single kernel dispatches (``oxh_time_next_launch``)."""

    def __init__(self):
        self.start, self.stop = _vp(), _vp()
        check(lib().oxh_event_create(ctypes.byref(self.start)))
        check(lib().oxh_event_create(ctypes.byref(self.stop)))

    def arm(self) -> None:
        """The calling thread's next kernel launch records this timer's events."""
        check(lib().oxh_time_next_launch(self.start, self.stop))

    def elapsed_ms(self) -> float:
        ms = _f32()
        check(lib().oxh_event_elapsed_ms(self.start, self.stop, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        if _lib is not None:
            _lib.oxh_event_destroy(self.start)
            _lib.oxh_event_destroy(self.stop)


def initialized_weights(shape, input_channels_per_group):
    """nn.rs:657-674 deterministic OIHW init (host memory), via the library."""
    import numpy as np

    dims = (_u64 * 4)(*[int(d) for d in shape])
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    check(lib().oxh_initialized_weights(dims, int(input_channels_per_group),
                                        out.ctypes.data_as(ctypes.POINTER(_f32))))
    return out.reshape(shape)


def checkpoint_save(path, tensors) -> None:
    """Writes an OXTR checkpoint (mobilenet_v4.rs:217-264); ``tensors`` is a sequence of
    (shape, float32 values) in order."""
    import numpy as np

    keep = []
    table = (CheckpointTensor * len(tensors))()
    for i, (shape, values) in enumerate(tensors):
        dims = np.ascontiguousarray(shape, dtype=np.uint64)
        vals = np.ascontiguousarray(values, dtype=np.float32).ravel()
        keep += [dims, vals]
        table[i] = CheckpointTensor(len(dims), dims.ctypes.data_as(ctypes.POINTER(_u64)),
                                    vals.size, vals.ctypes.data_as(ctypes.POINTER(_f32)))
    check(lib().oxh_checkpoint_save(str(path).encode(), table, len(tensors)))


def checkpoint_load(path) -> list:
    """Reads an OXTR checkpoint (mobilenet_v4.rs:386-428): a list of (shape tuple, float32
    values)."""
    import numpy as np

    handle = _vp()
    check(lib().oxh_checkpoint_load(str(path).encode(), ctypes.byref(handle)))
    try:
        count = _u64()
        check(lib().oxh_checkpoint_count(handle, ctypes.byref(count)))
        out = []
        for i in range(count.value):
            rank, n = _u64(), _u64()
            shape_p, data_p = ctypes.POINTER(_u64)(), ctypes.POINTER(_f32)()
            check(lib().oxh_checkpoint_entry(handle, i, ctypes.byref(rank), ctypes.byref(shape_p),
                                             ctypes.byref(n), ctypes.byref(data_p)))
            shape = tuple(shape_p[d] for d in range(rank.value))
            values = (np.ctypeslib.as_array(data_p, (n.value,)).copy() if n.value
                      else np.zeros(0, np.float32))
            out.append((shape, values))
        return out
    finally:
        lib().oxh_checkpoint_free(handle)


def conv2d_shape(batch, in_channels, height, width, out_channels, kernel, stride, padding,
                 groups) -> Conv2dShape:
    return Conv2dShape(batch, in_channels, height, width, out_channels, kernel, kernel, stride,
                       padding, groups)


def depthwise_conv_batch_norm_supported(shape: Conv2dShape) -> bool:
    """Whether the one-launch depthwise conv + BatchNorm entry points take this shape."""
    return bool(lib().oxh_depthwise_conv_batch_norm_supported(ctypes.byref(shape)))


def conv2d_output_size(shape: Conv2dShape) -> tuple[int, int]:
    oh, ow = _u64(), _u64()
    check(lib().oxh_conv2d_output_size(ctypes.byref(shape), ctypes.byref(oh), ctypes.byref(ow)))
    return oh.value, ow.value


def conv2d_forward_serial(shape: Conv2dShape) -> bool:
    """True when oxh_conv2d_forward sums each output in the CPU path's order (bit-identical),
    False when in another fixed order (four ordered parts over the input channels, or
    matrix-core sums) within 1e-5 * sum|terms| of it."""
    v = lib().oxh_conv2d_forward_serial(ctypes.byref(shape))
    if v < 0:
        raise OxideError(INVALID_SHAPE, "invalid conv2d shape")
    return bool(v)


def conv2d_input_backward_serial(shape: Conv2dShape) -> bool:
    """True when the input gradient sums each value in the CPU path's order (bit-identical),
    False when in another fixed order (four ordered parts over the output channels, or
    matrix-core sums) within 1e-5 * sum|terms| of it."""
    v = lib().oxh_conv2d_input_backward_serial(ctypes.byref(shape))
    if v < 0:
        raise OxideError(INVALID_SHAPE, "invalid conv2d shape")
    return bool(v)


def conv2d_workspace_size(shape: Conv2dShape) -> int:
    out = _u64()
    check(lib().oxh_conv2d_weight_backward_workspace_size(ctypes.byref(shape),
                                                          ctypes.byref(out)))
    return out.value


def init(device: int = 0) -> None:
    check(lib().oxh_init(device))


# ----------------------------------------------------------------------------- launchers

class LoadedModule:
    """Launchers with the reference kernel names (kernel_module.rs) over device tensors.

    Each call enqueues on ``stream`` (default: torch's current stream) and returns at once.
    Reductions use a workspace owned by this object, so calls through one module must be
    ordered on one stream.
    """

    def __init__(self, device: int = 0):
        init(device)
        self._bn_ws = Workspace()
        self._ce_ws = Workspace()
        self._conv_ws = Workspace()

    # -- elementwise (kernel_module.rs:8-34, 492-508, 1052-1059)
    def add(self, a, b, out, stream=None):
        check(lib().oxh_add(_stream(stream), _ptr(a), _ptr(b), _ptr(out), out.numel()))

    def mul(self, a, b, out, stream=None):
        check(lib().oxh_mul(_stream(stream), _ptr(a), _ptr(b), _ptr(out), out.numel()))

    def relu(self, x, out, stream=None):
        check(lib().oxh_relu(_stream(stream), _ptr(x), _ptr(out), out.numel()))

    def mul_backward(self, gradient, other, out, stream=None):
        check(lib().oxh_mul_backward(_stream(stream), _ptr(gradient), _ptr(other), _ptr(out),
                                     out.numel()))

    def relu_backward(self, gradient, x, out, stream=None):
        check(lib().oxh_relu_backward(_stream(stream), _ptr(gradient), _ptr(x), _ptr(out),
                                      out.numel()))

    def accumulate(self, a, b, out, stream=None):
        check(lib().oxh_accumulate(_stream(stream), _ptr(a), _ptr(b), _ptr(out), out.numel()))

    def elementwise_chain_forward(self, a, b, c, y, stream=None):
        check(lib().oxh_elementwise_chain_forward(_stream(stream), _ptr(a), _ptr(b), _ptr(c),
                                                  _ptr(y), y.numel()))

    def elementwise_chain_backward(self, a, b, c, gradient, da, db, dc, stream=None):
        check(lib().oxh_elementwise_chain_backward(_stream(stream), _ptr(a), _ptr(b), _ptr(c),
                                                   _ptr(gradient), _ptr(da), _ptr(db), _ptr(dc),
                                                   da.numel()))

    # -- batch norm (kernel_module.rs:827-964, 1061-1092)
    def _bn_ws_args(self, n, c, s):
        return self._bn_ws.ptr_bytes(batch_norm_workspace_size(n, c, s))

    def batch_norm_statistics(self, batch, channels, spatial, epsilon, x, mean, inverse_std,
                              unbiased_variance, stream=None):
        ws, wsb = self._bn_ws_args(batch, channels, spatial)
        check(lib().oxh_batch_norm_statistics(_stream(stream), batch, channels, spatial, epsilon,
                                              _ptr(x), _ptr(mean), _ptr(inverse_std),
                                              _ptr(unbiased_variance), ws, wsb))

    def batch_norm_update_running(self, momentum, batch_mean, batch_variance, old_mean,
                                  old_variance, new_mean, new_variance, stream=None):
        check(lib().oxh_batch_norm_update_running(_stream(stream), new_mean.numel(), momentum,
                                                  _ptr(batch_mean), _ptr(batch_variance),
                                                  _ptr(old_mean), _ptr(old_variance),
                                                  _ptr(new_mean), _ptr(new_variance)))

    def batch_norm_running_inverse_std(self, epsilon, variance, inverse_std, stream=None):
        check(lib().oxh_batch_norm_running_inverse_std(_stream(stream), variance.numel(),
                                                       epsilon, _ptr(variance),
                                                       _ptr(inverse_std)))

    def batch_norm_apply(self, channels, spatial, x, weight, bias, mean, inverse_std, out,
                         stream=None):
        batch = x.numel() // (channels * spatial)
        check(lib().oxh_batch_norm_apply(_stream(stream), batch, channels, spatial, _ptr(x),
                                         _ptr(weight), _ptr(bias), _ptr(mean),
                                         _ptr(inverse_std), _ptr(out)))

    def batch_norm_affine_backward(self, batch, channels, spatial, gradient, x, mean,
                                   inverse_std, weight_gradient, bias_gradient, stream=None):
        ws, wsb = self._bn_ws_args(batch, channels, spatial)
        check(lib().oxh_batch_norm_affine_backward(_stream(stream), batch, channels, spatial,
                                                   _ptr(gradient), _ptr(x), _ptr(mean),
                                                   _ptr(inverse_std), _ptr(weight_gradient),
                                                   _ptr(bias_gradient), ws, wsb))

    def batch_norm_input_backward(self, channels, spatial, samples, training, gradient, x,
                                  weight, mean, inverse_std, weight_gradient, bias_gradient,
                                  out, stream=None):
        batch = samples // spatial
        check(lib().oxh_batch_norm_input_backward(_stream(stream), batch, channels, spatial,
                                                  int(bool(training)), _ptr(gradient), _ptr(x),
                                                  _ptr(weight), _ptr(mean), _ptr(inverse_std),
                                                  _ptr(weight_gradient), _ptr(bias_gradient),
                                                  _ptr(out)))

    def batch_norm_forward_reduce(self, x, stream=None):
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_forward_reduce(_stream(stream), n, c, h * w, _ptr(x), ws,
                                                  wsb))

    def batch_norm_forward_apply(self, x, weight, bias, running_mean, running_variance,
                                 saved_mean, saved_inverse_std, out, momentum=0.1,
                                 epsilon=1e-5, stream=None):
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_forward_apply(_stream(stream), n, c, h * w, momentum, epsilon,
                                                 _ptr(x), _ptr(weight), _ptr(bias),
                                                 _ptr(running_mean), _ptr(running_variance),
                                                 _ptr(saved_mean), _ptr(saved_inverse_std),
                                                 _ptr(out), ws, wsb))

    def batch_norm_backward_reduce(self, gradient, x, saved_mean, saved_inverse_std,
                                   stream=None):
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_backward_reduce(_stream(stream), n, c, h * w, _ptr(gradient),
                                                   _ptr(x), _ptr(saved_mean),
                                                   _ptr(saved_inverse_std), ws, wsb))

    def batch_norm_backward_input(self, gradient, x, weight, saved_mean, saved_inverse_std,
                                  input_gradient, weight_gradient, bias_gradient, stream=None):
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_backward_input(_stream(stream), n, c, h * w, _ptr(gradient),
                                                  _ptr(x), _ptr(weight), _ptr(saved_mean),
                                                  _ptr(saved_inverse_std), _ptr(input_gradient),
                                                  _ptr(weight_gradient), _ptr(bias_gradient),
                                                  ws, wsb))

    def batch_norm_forward_train(self, x, weight, bias, running_mean, running_variance,
                                 saved_mean, saved_inverse_std, out, momentum=0.1, epsilon=1e-5,
                                 stream=None):
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_forward_train(_stream(stream), n, c, h * w, momentum, epsilon,
                                                 _ptr(x), _ptr(weight), _ptr(bias),
                                                 _ptr(running_mean), _ptr(running_variance),
                                                 _ptr(saved_mean), _ptr(saved_inverse_std),
                                                 _ptr(out), ws, wsb))

    def batch_norm_backward_train(self, gradient, x, weight, saved_mean, saved_inverse_std,
                                  input_gradient, weight_gradient, bias_gradient, stream=None):
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_backward_train(_stream(stream), n, c, h * w, _ptr(gradient),
                                                  _ptr(x), _ptr(weight), _ptr(saved_mean),
                                                  _ptr(saved_inverse_std), _ptr(input_gradient),
                                                  _ptr(weight_gradient), _ptr(bias_gradient),
                                                  ws, wsb))

    def batch_norm_relu_forward_train(self, x, weight, bias, running_mean, running_variance,
                                      saved_mean, saved_inverse_std, out, momentum=0.1,
                                      epsilon=1e-5, stream=None):
        """out = relu(batch_norm(x)) (ConvNormAct with activation, nn.rs:376-385)."""
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_relu_forward_train(
            _stream(stream), n, c, h * w, momentum, epsilon, _ptr(x), _ptr(weight), _ptr(bias),
            _ptr(running_mean), _ptr(running_variance), _ptr(saved_mean),
            _ptr(saved_inverse_std), _ptr(out), ws, wsb))

    def batch_norm_relu_backward_train(self, gradient, out, x, weight, saved_mean,
                                       saved_inverse_std, input_gradient, weight_gradient,
                                       bias_gradient, stream=None):
        """Backward of batch_norm_relu_forward_train; ``gradient`` is w.r.t. its output
        ``out``."""
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_relu_backward_train(
            _stream(stream), n, c, h * w, _ptr(gradient), _ptr(out), _ptr(x), _ptr(weight),
            _ptr(saved_mean), _ptr(saved_inverse_std), _ptr(input_gradient),
            _ptr(weight_gradient), _ptr(bias_gradient), ws, wsb))

    def batch_norm_add_forward_train(self, x, weight, bias, running_mean, running_variance,
                                     saved_mean, saved_inverse_std, addend, out, momentum=0.1,
                                     epsilon=1e-5, stream=None):
        """BatchNorm training forward followed by the residual add: ``out`` = BN(x) + addend."""
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_batch_norm_add_forward_train(
            _stream(stream), n, c, h * w, momentum, epsilon, _ptr(x), _ptr(weight), _ptr(bias),
            _ptr(running_mean), _ptr(running_variance), _ptr(saved_mean),
            _ptr(saved_inverse_std), _ptr(addend), _ptr(out), ws, wsb))

    def conv_batch_norm_backward_train(self, gradient, relu_out, x, weight, saved_mean,
                                       saved_inverse_std, input_gradient, weight_gradient,
                                       bias_gradient, conv_bias_gradient, stream=None):
        """BatchNorm training backward (through the following ReLU when ``relu_out`` is not
        None) that also writes the per-channel sum of ``input_gradient``: the bias gradient of
        the convolution producing ``x``."""
        n, c, h, w = x.shape
        ws, wsb = self._bn_ws_args(n, c, h * w)
        check(lib().oxh_conv_batch_norm_backward_train(
            _stream(stream), n, c, h * w, _ptr(gradient), _ptr(relu_out), _ptr(x),
            _ptr(weight), _ptr(saved_mean), _ptr(saved_inverse_std), _ptr(input_gradient),
            _ptr(weight_gradient), _ptr(bias_gradient), _ptr(conv_bias_gradient), ws, wsb))

    # -- cross entropy (kernel_module.rs:966-1050)
    def cross_entropy_forward(self, batch, classes, logits, targets, loss, error_flag=None,
                              stream=None):
        ws, wsb = self._ce_ws.ptr_bytes(cross_entropy_workspace_size(batch, classes))
        check(lib().oxh_cross_entropy_forward(_stream(stream), batch, classes, _ptr(logits),
                                              _ptr(targets), _ptr(loss), _ptr(error_flag), ws,
                                              wsb))

    def cross_entropy_backward(self, batch, classes, logits, targets, outer_gradient, grad,
                               error_flag=None, stream=None):
        check(lib().oxh_cross_entropy_backward(_stream(stream), batch, classes, _ptr(logits),
                                               _ptr(targets), _ptr(outer_gradient), _ptr(grad),
                                               _ptr(error_flag)))

    def cross_entropy_forward_backward(self, batch, classes, logits, targets, outer_gradient,
                                       loss, grad, error_flag=None, stream=None):
        ws, wsb = self._ce_ws.ptr_bytes(cross_entropy_workspace_size(batch, classes))
        check(lib().oxh_cross_entropy_forward_backward(_stream(stream), batch, classes,
                                                       _ptr(logits), _ptr(targets),
                                                       _ptr(outer_gradient), _ptr(loss),
                                                       _ptr(grad), _ptr(error_flag), ws, wsb))

    # -- AdamW (kernel_module.rs:1094-1127)
    def adamw(self, learning_rate, weight_decay, beta1, beta2, first_correction,
              second_correction, epsilon, parameter, gradient, first_moment, second_moment,
              new_parameter, new_first_moment, new_second_moment, stream=None):
        check(lib().oxh_adamw(_stream(stream), learning_rate, weight_decay, beta1, beta2,
                              first_correction, second_correction, epsilon, _ptr(parameter),
                              _ptr(gradient), _ptr(first_moment), _ptr(second_moment),
                              _ptr(new_parameter), _ptr(new_first_moment),
                              _ptr(new_second_moment), parameter.numel()))

    def adamw_multi_tensor(self, learning_rate, weight_decay, beta1, beta2, first_correction,
                           second_correction, epsilon, tensors, stream=None):
        """``tensors``: sequence of (parameter, gradient, first_moment, second_moment)."""
        table = (AdamWTensor * len(tensors))()
        for i, (p, g, m, v) in enumerate(tensors):
            table[i] = AdamWTensor(_ptr(p), _ptr(g), _ptr(m), _ptr(v), p.numel())
        check(lib().oxh_adamw_multi_tensor(_stream(stream), learning_rate, weight_decay, beta1,
                                           beta2, first_correction, second_correction, epsilon,
                                           table, len(tensors)))

    def adamw_multi_tensor_step(self, learning_rate, weight_decay, beta1, beta2, epsilon,
                                step_counter, tensors, stream=None):
        """``tensors``: sequence of (parameter, gradient, first_moment, second_moment);
        ``step_counter``: device int32 incremented before the update."""
        table = (AdamWTensor * len(tensors))()
        for i, (p, g, m, v) in enumerate(tensors):
            table[i] = AdamWTensor(_ptr(p), _ptr(g), _ptr(m), _ptr(v), p.numel())
        check(lib().oxh_adamw_multi_tensor_step(_stream(stream), learning_rate, weight_decay,
                                                beta1, beta2, epsilon, _ptr(step_counter),
                                                table, len(tensors)))

    def adamw_table_step(self, learning_rate, weight_decay, beta1, beta2, epsilon, step_counter,
                         tensors, stream=None):
        """The device-table variant: the table and its chunk starts are copied to the device
        (kept alive on the returned object until the launch completes)."""
        import torch

        count = len(tensors)
        table = (AdamWTensor * count)()
        for i, (p, g, m, v) in enumerate(tensors):
            table[i] = AdamWTensor(_ptr(p), _ptr(g), _ptr(m), _ptr(v), p.numel())
        starts = (_u32 * (count + 1))()
        total = _u64()
        check(lib().oxh_adamw_table_layout(table, count, starts, ctypes.byref(total)))
        dev_table = torch.frombuffer(bytearray(bytes(table)), dtype=torch.uint8).to(
            step_counter.device)
        dev_starts = torch.tensor(list(starts), dtype=torch.int32, device=step_counter.device)
        torch.cuda.synchronize()
        check(lib().oxh_adamw_multi_tensor_table_step(
            _stream(stream), learning_rate, weight_decay, beta1, beta2, epsilon,
            _ptr(step_counter), dev_table.data_ptr(), dev_starts.data_ptr(),
            count, total.value))
        return dev_table, dev_starts

    # -- conv2d / avg_pool2d (kernel_module.rs:359-490, 558-825)
    def conv2d_forward(self, shape, x, weight, bias, out, stream=None):
        check(lib().oxh_conv2d_forward(_stream(stream), ctypes.byref(shape), _ptr(x),
                                       _ptr(weight), _ptr(bias), _ptr(out)))

    def conv2d_input_backward(self, shape, gradient, weight, input_gradient, stream=None):
        check(lib().oxh_conv2d_input_backward(_stream(stream), ctypes.byref(shape),
                                              _ptr(gradient), _ptr(weight),
                                              _ptr(input_gradient)))

    def conv2d_input_backward_accumulate(self, shape, gradient, weight, addend, input_gradient,
                                         stream=None):
        """input_gradient = conv2d input backward + addend (gradient accumulation)."""
        check(lib().oxh_conv2d_input_backward_accumulate(_stream(stream), ctypes.byref(shape),
                                                         _ptr(gradient), _ptr(weight),
                                                         _ptr(addend), _ptr(input_gradient)))

    def conv2d_weight_backward(self, shape, gradient, x, weight_gradient, stream=None):
        ws, wsb = self._conv_ws.ptr_bytes(conv2d_workspace_size(shape))
        check(lib().oxh_conv2d_weight_backward(_stream(stream), ctypes.byref(shape),
                                               _ptr(gradient), _ptr(x), _ptr(weight_gradient),
                                               ws, wsb))

    def conv2d_backward(self, shape, gradient, x, weight, input_gradient, weight_gradient,
                        bias_gradient=None, addend=None, stream=None):
        """The whole conv VJP: weight, optional bias and input gradients in one call
        (input_gradient None: the parameter gradients only)."""
        ws, wsb = self._conv_ws.ptr_bytes(conv2d_workspace_size(shape))
        check(lib().oxh_conv2d_backward(
            _stream(stream), ctypes.byref(shape), _ptr(gradient), _ptr(x), _ptr(weight),
            _ptr(addend), _ptr(input_gradient), _ptr(weight_gradient), _ptr(bias_gradient),
            ws, wsb))

    def conv2d_bias_backward(self, shape, gradient, bias_gradient, stream=None):
        ws, wsb = self._conv_ws.ptr_bytes(conv2d_workspace_size(shape))
        check(lib().oxh_conv2d_bias_backward(_stream(stream), ctypes.byref(shape),
                                             _ptr(gradient), _ptr(bias_gradient), ws, wsb))

    def depthwise_conv_batch_norm_forward_train(self, shape, relu, momentum, epsilon, x,
                                                conv_weight, conv_bias, conv_out, bn_weight,
                                                bn_bias, running_mean, running_variance,
                                                saved_mean, saved_inverse_std, out,
                                                stream=None):
        """Depthwise conv2d + BatchNorm2d training forward (+ ReLU) in one launch."""
        check(lib().oxh_depthwise_conv_batch_norm_forward_train(
            _stream(stream), ctypes.byref(shape), int(relu), momentum, epsilon, _ptr(x),
            _ptr(conv_weight), _ptr(conv_bias), _ptr(conv_out), _ptr(bn_weight), _ptr(bn_bias),
            _ptr(running_mean), _ptr(running_variance), _ptr(saved_mean),
            _ptr(saved_inverse_std), _ptr(out)))

    def depthwise_conv_batch_norm_backward_train(self, shape, gradient, relu_out, conv_out,
                                                 bn_weight, saved_mean, saved_inverse_std, x,
                                                 conv_weight, addend, conv_out_gradient,
                                                 bn_weight_gradient, bn_bias_gradient,
                                                 conv_bias_gradient, conv_weight_gradient,
                                                 input_gradient, stream=None):
        """Its backward in one launch (``relu_out``, ``addend``, ``conv_out_gradient`` and
        ``input_gradient`` may be None)."""
        check(lib().oxh_depthwise_conv_batch_norm_backward_train(
            _stream(stream), ctypes.byref(shape), _ptr(gradient), _ptr(relu_out),
            _ptr(conv_out), _ptr(bn_weight), _ptr(saved_mean), _ptr(saved_inverse_std), _ptr(x),
            _ptr(conv_weight), _ptr(addend), _ptr(conv_out_gradient), _ptr(bn_weight_gradient),
            _ptr(bn_bias_gradient), _ptr(conv_bias_gradient), _ptr(conv_weight_gradient),
            _ptr(input_gradient)))

    def batch_norm_depthwise_conv_batch_norm_forward_train(self, shape, pre, layer,
                                                           stream=None):
        """A BatchNorm (+ ReLU) feeding a depthwise ConvNormAct, in one launch with it.
        ``pre``: dict relu, momentum, epsilon, x, weight, bias, residual (optional),
        running_mean, running_variance, saved_mean, saved_inverse_std, out; ``layer``: dict
        relu, momentum,
        epsilon, conv_weight, conv_bias, conv_out, weight, bias, running_mean,
        running_variance, saved_mean, saved_inverse_std, out."""
        p, q = pre, layer
        check(lib().oxh_batch_norm_depthwise_conv_batch_norm_forward_train(
            _stream(stream), ctypes.byref(shape), int(p["relu"]), p["momentum"], p["epsilon"],
            _ptr(p["x"]), _ptr(p["weight"]), _ptr(p["bias"]), _ptr(p.get("residual")),
            *[_ptr(p[k]) for k in ("running_mean", "running_variance", "saved_mean",
                                   "saved_inverse_std", "out")],
            int(q["relu"]), q["momentum"], q["epsilon"],
            *[_ptr(q[k]) for k in ("conv_weight", "conv_bias", "conv_out", "weight", "bias",
                                   "running_mean", "running_variance", "saved_mean",
                                   "saved_inverse_std", "out")]))

    def batch_norm_depthwise_conv_batch_norm_backward_train(self, shape, layer, pre,
                                                            stream=None):
        """Its backward.  ``layer``: dict gradient, relu_out (or None), conv_out, weight,
        saved_mean, saved_inverse_std, conv_in, conv_weight, addend and conv_in_gradient
        (optional), conv_out_gradient (or None), weight_gradient, bias_gradient,
        conv_bias_gradient, conv_weight_gradient; ``pre``:
        dict relu, x, weight, saved_mean, saved_inverse_std, weight_gradient, bias_gradient,
        input_gradient, input_gradient_sum (or None)."""
        q, p = layer, pre
        check(lib().oxh_batch_norm_depthwise_conv_batch_norm_backward_train(
            _stream(stream), ctypes.byref(shape),
            *[_ptr(q[k]) for k in ("gradient", "relu_out", "conv_out", "weight", "saved_mean",
                                   "saved_inverse_std", "conv_in", "conv_weight")],
            _ptr(q.get("addend")), int(p["relu"]),
            *[_ptr(p[k]) for k in ("x", "weight", "saved_mean", "saved_inverse_std")],
            *[_ptr(q[k]) for k in ("conv_out_gradient", "weight_gradient", "bias_gradient",
                                   "conv_bias_gradient", "conv_weight_gradient")],
            _ptr(q.get("conv_in_gradient")),
            *[_ptr(p[k]) for k in ("weight_gradient", "bias_gradient", "input_gradient",
                                   "input_gradient_sum")]))

    def avg_pool2d_forward(self, shape, x, out, stream=None):
        check(lib().oxh_avg_pool2d_forward(_stream(stream), ctypes.byref(shape), _ptr(x),
                                           _ptr(out)))

    def avg_pool2d_backward(self, shape, gradient, input_gradient, stream=None):
        check(lib().oxh_avg_pool2d_backward(_stream(stream), ctypes.byref(shape),
                                            _ptr(gradient), _ptr(input_gradient)))

    def argmax_rows(self, logits, indices, stream=None):
        rows, classes = logits.shape
        check(lib().oxh_argmax_rows(_stream(stream), rows, classes, _ptr(logits),
                                    _ptr(indices)))


def load_kernels(device: int = 0) -> LoadedModule:
    """``oxide_torch_cuda::load_kernels`` (lib.rs:19-30): the module for ``device``."""
    return LoadedModule(device)


# ----------------------------------------------------------------------------- graphs

class HipGraphExec:
    """``CudaGraphExec`` (cuda_graph.rs:30-179): capture once, launch many times."""

    def __init__(self, handle: int):
        self._handle = handle

    @classmethod
    def capture(cls, stream, record: Callable[[], None]) -> "HipGraphExec":
        s = _stream(stream)
        check(lib().oxh_graph_begin(s))
        try:
            record()
        except Exception as exc:
            # cuda_graph.rs:84-97: end and discard the capture, keep the stream usable.
            lib().oxh_graph_abort(s)
            if isinstance(exc, OxideError):
                raise OxideError(EXECUTION, f"graph recording failed: {exc}") from exc
            raise OxideError(EXECUTION, f"graph recording failed: {exc}") from exc
        handle = _vp()
        check(lib().oxh_graph_end(s, ctypes.byref(handle)))
        return cls(handle.value)

    def launch(self, stream) -> None:
        check(lib().oxh_graph_launch(self._handle, _stream(stream)))

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.oxh_graph_destroy(self._handle)
            self._handle = None
