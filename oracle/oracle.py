"""ctypes front end of the CPU oracle (oracle/liboxide_oracle.so).

TEST INFRASTRUCTURE ONLY.  The oracle restates oxide-torch's CPU path (tuna2134/oxide-beta,
crates/oxide-torch/src/tensor/{evaluation,autograd}.rs, optim.rs, nn.rs) and is the checker for
the HIP kernels.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module; the product never does.

Every wrapper takes and returns C-contiguous float32 numpy arrays and raises ``OracleError``
carrying the reference's error kind where the reference returns an ``Err``.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "liboxide_oracle.so"

OK = 0
INVALID_SHAPE = 1
EXECUTION = 2
_KIND = {INVALID_SHAPE: "InvalidShape", EXECUTION: "Execution"}


class OracleError(RuntimeError):
    def __init__(self, code: int):
        self.kind = _KIND.get(code, f"status {code}")
        super().__init__(self.kind)


_F = ctypes.POINTER(ctypes.c_float)
_U64P = ctypes.POINTER(ctypes.c_uint64)
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float
_i32 = ctypes.c_int32
_int = ctypes.c_int

_SIGNATURES = {
    "oro_add": (None, [_F, _F, _F, _u64]),
    "oro_mul": (None, [_F, _F, _F, _u64]),
    "oro_relu": (None, [_F, _F, _u64]),
    "oro_mul_backward": (None, [_F, _F, _F, _u64]),
    "oro_relu_backward": (None, [_F, _F, _F, _u64]),
    "oro_accumulate": (None, [_F, _F, _u64]),
    "oro_chain_forward": (None, [_F, _F, _F, _F, _u64]),
    "oro_chain_backward_ones": (None, [_F, _F, _F, _F, _F, _F, _u64]),
    "oro_bn_batch_statistics": (_int, [_F, _u64, _u64, _u64, _f32, _F, _F]),
    "oro_bn_update_running": (_int, [_F, _u64, _u64, _u64, _f32, _F, _F]),
    "oro_bn_running_statistics": (None, [_F, _u64, _f32, _F]),
    "oro_bn_apply": (None, [_F, _u64, _u64, _u64, _F, _F, _F, _F, _F]),
    "oro_bn_forward": (_int, [_F, _u64, _u64, _u64, _F, _F, _F, _F, _int, _f32, _f32, _F, _F, _F]),
    "oro_bn_backward": (None, [_F, _F, _u64, _u64, _u64, _F, _F, _F, _int, _F, _F, _F]),
    "oro_class_index": (_int, [_f32, _u64, _U64P]),
    "oro_ce_forward": (_int, [_F, _F, _u64, _u64, _F]),
    "oro_ce_backward": (_int, [_F, _F, _u64, _u64, _f32, _F]),
    "oro_powi": (_f32, [_f32, _i32]),
    "oro_adamw_update": (None, [_F, _F, _F, _F, _u64, _f32, _f32, _f32, _f32, _f32, _i32]),
    "oro_conv2d_forward": (None, [_F, _F, _F] + [_u64] * 10 + [_F]),
    "oro_conv2d_backward": (None, [_F, _F, _F] + [_u64] * 10 + [_F, _F, _F]),
    "oro_avg_pool2d_forward": (None, [_F] + [_u64] * 8 + [_F]),
    "oro_avg_pool2d_backward": (None, [_F] + [_u64] * 8 + [_F]),
    "oro_initialized_weights": (None, [_U64P, _u64, _F]),
    "oro_argmax_rows": (None, [_F, _u64, _u64, _U64P]),
    "oro_mnist_normalize": (None, [ctypes.c_void_p, _u64, _F]),
    "oro_mnist_shuffle": (None, [_U64P, _u64]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is not built; run `make -C oracle` or __graft_entry__.build()")
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous, "oracle needs contiguous float32"
    return a.ctypes.data_as(_F)


def _c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(code: int) -> None:
    if code != OK:
        raise OracleError(code)


# ---------------------------------------------------------------- elementwise

def add(a, b):
    a, b = _c(a), _c(b)
    out = np.empty_like(a)
    lib().oro_add(_f(a), _f(b), _f(out), a.size)
    return out


def mul(a, b):
    a, b = _c(a), _c(b)
    out = np.empty_like(a)
    lib().oro_mul(_f(a), _f(b), _f(out), a.size)
    return out


def relu(x):
    x = _c(x)
    out = np.empty_like(x)
    lib().oro_relu(_f(x), _f(out), x.size)
    return out


def mul_backward(grad, other):
    grad, other = _c(grad), _c(other)
    out = np.empty_like(grad)
    lib().oro_mul_backward(_f(grad), _f(other), _f(out), grad.size)
    return out


def relu_backward(grad, inp):
    grad, inp = _c(grad), _c(inp)
    out = np.empty_like(grad)
    lib().oro_relu_backward(_f(grad), _f(inp), _f(out), grad.size)
    return out


def accumulate(current, incoming):
    out = _c(current).copy()
    incoming = _c(incoming)
    lib().oro_accumulate(_f(out), _f(incoming), out.size)
    return out


def chain_forward(a, b, c):
    a, b, c = _c(a), _c(b), _c(c)
    y = np.empty_like(a)
    lib().oro_chain_forward(_f(a), _f(b), _f(c), _f(y), a.size)
    return y


def chain_backward_ones(a, b, c):
    a, b, c = _c(a), _c(b), _c(c)
    da, db, dc = np.empty_like(a), np.empty_like(a), np.empty_like(a)
    lib().oro_chain_backward_ones(_f(a), _f(b), _f(c), _f(da), _f(db), _f(dc), a.size)
    return da, db, dc


# ---------------------------------------------------------------- batch norm

def bn_batch_statistics(x, epsilon):
    x = _c(x)
    n, c, h, w = x.shape
    mean = np.empty(c, np.float32)
    inv_std = np.empty(c, np.float32)
    _check(lib().oro_bn_batch_statistics(_f(x), n, c, h * w, epsilon, _f(mean), _f(inv_std)))
    return mean, inv_std


def bn_forward(x, weight, bias, running_mean, running_var, training=True, momentum=0.1,
               epsilon=1e-5):
    """Returns (y, saved_mean, saved_inv_std, new_running_mean, new_running_var)."""
    x = _c(x)
    n, c, h, w = x.shape
    weight, bias = _c(weight), _c(bias)
    rm, rv = _c(running_mean).copy(), _c(running_var).copy()
    y = np.empty_like(x)
    mean = np.empty(c, np.float32)
    inv_std = np.empty(c, np.float32)
    _check(lib().oro_bn_forward(_f(x), n, c, h * w, _f(weight), _f(bias), _f(rm), _f(rv),
                                int(bool(training)), momentum, epsilon, _f(y), _f(mean),
                                _f(inv_std)))
    return y, mean, inv_std, rm, rv


def bn_backward(grad, x, weight, mean, inv_std, training=True):
    """Returns (dx, dweight, dbias)."""
    grad, x = _c(grad), _c(x)
    n, c, h, w = x.shape
    weight, mean, inv_std = _c(weight), _c(mean), _c(inv_std)
    dx = np.empty_like(x)
    dw = np.empty(c, np.float32)
    db = np.empty(c, np.float32)
    lib().oro_bn_backward(_f(grad), _f(x), n, c, h * w, _f(weight), _f(mean), _f(inv_std),
                          int(bool(training)), _f(dx), _f(dw), _f(db))
    return dx, dw, db


# ---------------------------------------------------------------- cross entropy

def class_index(value, classes):
    out = ctypes.c_uint64()
    _check(lib().oro_class_index(float(value), classes, ctypes.byref(out)))
    return out.value


def ce_forward(logits, targets):
    logits, targets = _c(logits), _c(targets)
    b, k = logits.shape
    loss = np.empty(1, np.float32)
    _check(lib().oro_ce_forward(_f(logits), _f(targets), b, k, _f(loss)))
    return float(loss[0])


def ce_backward(logits, targets, outer=1.0):
    logits, targets = _c(logits), _c(targets)
    b, k = logits.shape
    grad = np.empty_like(logits)
    _check(lib().oro_ce_backward(_f(logits), _f(targets), b, k, outer, _f(grad)))
    return grad


# ---------------------------------------------------------------- AdamW

def powi(a, b):
    return float(lib().oro_powi(a, b))


def adamw_update(param, grad, m, v, step, lr=1e-3, weight_decay=0.01, beta1=0.9, beta2=0.999,
                 epsilon=1e-8):
    """One update at optimizer step ``step``; returns new (param, m, v)."""
    p = _c(param).copy()
    m = _c(m).copy()
    v = _c(v).copy()
    g = _c(grad)
    lib().oro_adamw_update(_f(p), _f(g), _f(m), _f(v), p.size, lr, weight_decay, beta1, beta2,
                           epsilon, step)
    return p, m, v


# ---------------------------------------------------------------- conv2d / avg_pool2d

def conv2d_forward(x, weight, bias, stride, padding, groups):
    x, weight, bias = _c(x), _c(weight), _c(bias)
    n, cin, h, w = x.shape
    cout, _, kh, kw = weight.shape
    oh, ow = (h + 2 * padding - kh) // stride + 1, (w + 2 * padding - kw) // stride + 1
    out = np.empty((n, cout, oh, ow), np.float32)
    lib().oro_conv2d_forward(_f(x), _f(weight), _f(bias), n, cin, h, w, cout, kh, kw, stride,
                             padding, groups, _f(out))
    return out


def conv2d_backward(grad, x, weight, stride, padding, groups):
    """Returns (dinput, dweight, dbias)."""
    grad, x, weight = _c(grad), _c(x), _c(weight)
    n, cin, h, w = x.shape
    cout, _, kh, kw = weight.shape
    dx = np.empty_like(x)
    dw = np.empty_like(weight)
    db = np.empty(cout, np.float32)
    lib().oro_conv2d_backward(_f(grad), _f(x), _f(weight), n, cin, h, w, cout, kh, kw, stride,
                              padding, groups, _f(dx), _f(dw), _f(db))
    return dx, dw, db


def conv2d_bias_backward(grad):
    """Bias gradient of a convolution with output gradient ``grad`` [n, c, h, w]: the dbias of
    oro_conv2d_backward (evaluation of autograd.rs:412-527's bias sum), which does not depend
    on the input or weights -- run on a 1x1, one-input-channel geometry of the same output."""
    grad = _c(grad)
    n, c, h, w = grad.shape
    return conv2d_backward(grad, np.zeros((n, 1, h, w), np.float32),
                           np.zeros((c, 1, 1, 1), np.float32), 1, 0, 1)[2]


def avg_pool2d_forward(x, kernel, stride):
    x = _c(x)
    n, c, h, w = x.shape
    oh, ow = (h - kernel[0]) // stride[0] + 1, (w - kernel[1]) // stride[1] + 1
    out = np.empty((n, c, oh, ow), np.float32)
    lib().oro_avg_pool2d_forward(_f(x), n, c, h, w, kernel[0], kernel[1], stride[0], stride[1],
                                 _f(out))
    return out


def avg_pool2d_backward(grad, input_shape, kernel, stride):
    grad = _c(grad)
    n, c, h, w = input_shape
    dx = np.empty(input_shape, np.float32)
    lib().oro_avg_pool2d_backward(_f(grad), n, c, h, w, kernel[0], kernel[1], stride[0],
                                  stride[1], _f(dx))
    return dx


# ---------------------------------------------------------------- model helpers

def initialized_weights(shape, input_channels_per_group):
    shape_arr = np.ascontiguousarray(shape, dtype=np.uint64)
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().oro_initialized_weights(shape_arr.ctypes.data_as(_U64P), input_channels_per_group,
                                  _f(out))
    return out.reshape(shape)


def argmax_rows(logits):
    logits = _c(logits)
    rows, classes = logits.shape
    out = np.empty(rows, np.uint64)
    lib().oro_argmax_rows(_f(logits), rows, classes, out.ctypes.data_as(_U64P))
    return out


# ---------------------------------------------------------------- MNIST data

def mnist_normalize(pixels):
    """mnist.rs:118-121 per byte, float32."""
    pixels = np.ascontiguousarray(pixels, dtype=np.uint8)
    out = np.empty(pixels.shape, np.float32)
    lib().oro_mnist_normalize(pixels.ctypes.data, pixels.size, _f(out))
    return out


def mnist_order(count, shuffle):
    """MnistBatches::new index order (mnist.rs:84-100,191-199)."""
    values = np.arange(count, dtype=np.uint64)
    if shuffle:
        lib().oro_mnist_shuffle(values.ctypes.data_as(_U64P), count)
    return values


# ---------------------------------------------------------------- OXTR checkpoints

def oxtr_bytes(tensors):
    """mobilenet_v4.rs:217-264: the bytes save() writes for (shape, values) pairs."""
    import struct

    out = [b"OXTR\x01", struct.pack("<Q", len(tensors))]
    for shape, values in tensors:
        values = np.ascontiguousarray(values, dtype=np.float32).ravel()
        out.append(struct.pack("<Q", len(shape)))
        out.extend(struct.pack("<Q", int(d)) for d in shape)
        out.append(struct.pack("<Q", values.size))
        out.append(values.astype("<f4").tobytes())
    return b"".join(out)
