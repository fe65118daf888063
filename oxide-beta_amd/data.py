"""MNIST IDX data (crates/oxide-torch/src/data/mnist.rs) through liboxide_hip.so.

``Mnist.load(directory)`` reads and validates the four canonical uncompressed IDX files in the
library (C++); ``train_batches`` / ``test_batches`` mirror ``MnistBatches`` (index order from
the reference's deterministic shuffle, last batch short, images normalized as
(pixel / 255 - 0.1307) / 0.3081 in fp32, labels as fp32) on the host; ``DeviceSplit`` keeps a
split's bytes in device memory and gathers + normalizes a batch on the GPU straight into a
training step's input and target buffers (the same values, bit for bit).
"""

from __future__ import annotations

import ctypes

import numpy as np

import oxide_hip as ox

PIXELS = 28 * 28


def parse_images(data: bytes) -> int:
    """parse_images (mnist.rs:145-170): the image count of a valid IDX image file."""
    buf = np.frombuffer(data, dtype=np.uint8)
    count = ctypes.c_uint64()
    ox.check(ox.lib().oxh_idx_parse_images(buf.ctypes.data if buf.size else None, buf.size,
                                           ctypes.byref(count)))
    return count.value


def parse_labels(data: bytes) -> int:
    """parse_labels (mnist.rs:172-183): the label count of a valid IDX label file."""
    buf = np.frombuffer(data, dtype=np.uint8)
    count = ctypes.c_uint64()
    ox.check(ox.lib().oxh_idx_parse_labels(buf.ctypes.data if buf.size else None, buf.size,
                                           ctypes.byref(count)))
    return count.value


def batch_order(count: int, shuffle: bool) -> np.ndarray:
    """MnistBatches::new's index order: 0..count-1, shuffled by deterministic_shuffle
    (mnist.rs:191-199) when ``shuffle``."""
    out = np.empty(count, dtype=np.uint64)
    ox.check(ox.lib().oxh_mnist_batch_order(count, int(bool(shuffle)),
                                            out.ctypes.data if count else None))
    return out


def host_batch(images: np.ndarray, labels: np.ndarray, indices: np.ndarray):
    """One normalized batch on the host (MnistBatches::next, mnist.rs:103-133):
    images [b, 1, 28, 28] float32, labels [b] float32."""
    images = np.ascontiguousarray(images, dtype=np.uint8)
    labels = np.ascontiguousarray(labels, dtype=np.uint8)
    idx = np.ascontiguousarray(indices, dtype=np.uint64)
    out_images = np.empty((idx.size, 1, 28, 28), np.float32)
    out_labels = np.empty(idx.size, np.float32)
    ox.check(ox.lib().oxh_mnist_batch_host(images.ctypes.data, labels.ctypes.data, labels.size,
                                           idx.ctypes.data, idx.size, out_images.ctypes.data,
                                           out_labels.ctypes.data))
    return out_images, out_labels


class MnistBatches:
    """Iterator over (images, labels) batches of one split (mnist.rs:78-133)."""

    def __init__(self, images, labels, batch_size: int, shuffle: bool):
        if batch_size == 0:
            raise ox.OxideError(ox.INVALID_SHAPE, "batch_size must be non-zero")
        self.images, self.labels = images, labels
        self.indices = batch_order(labels.size, shuffle)
        self.position, self.batch_size = 0, batch_size

    def __iter__(self):
        return self

    def __next__(self):
        if self.position >= self.indices.size:
            raise StopIteration
        end = min(self.position + self.batch_size, self.indices.size)
        chunk = self.indices[self.position:end]
        self.position = end
        return host_batch(self.images, self.labels, chunk)


class Mnist:
    """The four canonical IDX files of ``directory`` (Mnist::load, mnist.rs:26-49)."""

    def __init__(self, handle: int):
        self._handle = handle
        self.train_images, self.train_labels = self._split(0)
        self.test_images, self.test_labels = self._split(1)

    @classmethod
    def load(cls, directory) -> "Mnist":
        handle = ctypes.c_void_p()
        ox.check(ox.lib().oxh_mnist_load(str(directory).encode(), ctypes.byref(handle)))
        return cls(handle.value)

    def _split(self, test: int):
        images, labels, count = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_uint64()
        ox.check(ox.lib().oxh_mnist_split(self._handle, test, ctypes.byref(images),
                                          ctypes.byref(labels), ctypes.byref(count)))
        n = count.value
        if n == 0:
            return np.zeros((0, PIXELS), np.uint8), np.zeros(0, np.uint8)
        im = np.ctypeslib.as_array(ctypes.cast(images, ctypes.POINTER(ctypes.c_uint8)),
                                   (n * PIXELS,)).reshape(n, PIXELS).copy()
        lb = np.ctypeslib.as_array(ctypes.cast(labels, ctypes.POINTER(ctypes.c_uint8)),
                                   (n,)).copy()
        return im, lb

    def train_len(self) -> int:
        return self.train_labels.size

    def test_len(self) -> int:
        return self.test_labels.size

    def train_batches(self, batch_size: int, shuffle: bool) -> MnistBatches:
        return MnistBatches(self.train_images, self.train_labels, batch_size, shuffle)

    def test_batches(self, batch_size: int) -> MnistBatches:
        return MnistBatches(self.test_images, self.test_labels, batch_size, False)

    def __del__(self):
        if getattr(self, "_handle", None) and ox._lib is not None:
            ox._lib.oxh_mnist_free(self._handle)
            self._handle = None


class DeviceSplit:
    """One split resident in device memory with its batch order; ``gather`` writes batch
    ``k`` (positions k*b .. k*b+b-1 of the order) into device image / label buffers."""

    def __init__(self, images: np.ndarray, labels: np.ndarray, shuffle: bool, device: int = 0):
        import torch

        if labels.size >= 2 ** 31:
            raise ox.OxideError(ox.INVALID_SHAPE, "a split is limited to 2^31 images")
        dev = torch.device(f"cuda:{device}")
        self.count = labels.size
        self.images = torch.from_numpy(np.ascontiguousarray(images, np.uint8).ravel()).to(dev)
        self.labels = torch.from_numpy(np.ascontiguousarray(labels, np.uint8)).to(dev)
        order = batch_order(self.count, shuffle)
        self.order_host = order
        self.order = torch.from_numpy(order.astype(np.int32)).to(dev)  # uint32 bit pattern
        torch.cuda.synchronize()

    def batches(self, batch_size: int) -> int:
        """Full batches in one pass (a fixed-shape step drops the short last batch)."""
        return self.count // batch_size

    def gather(self, k: int, batch_size: int, out_images, out_labels, stream=None) -> None:
        first = k * batch_size
        if first + batch_size > self.count:
            raise ox.OxideError(ox.INVALID_SHAPE, "batch beyond the split")
        if out_images.numel() != batch_size * PIXELS or out_labels.numel() != batch_size:
            raise ox.OxideError(ox.INVALID_SHAPE, "output buffers do not match the batch")
        ox.check(ox.lib().oxh_mnist_gather_batch(
            ox._stream(stream), self.images.data_ptr(), self.labels.data_ptr(), self.count,
            self.order.data_ptr() + 4 * first, batch_size, out_images.data_ptr(),
            out_labels.data_ptr()))
