"""MNIST IDX data (crates/oxide-torch/src/data/mnist.rs) and OXTR checkpoints
(mobilenet_v4.rs:217-264,266-321,386-428) on the host: the library's C++ against the oracle and
the reference's own tests and error rules (no GPU)."""

import struct

import numpy as np
import pytest

import data as D
import oracle
import oxide_hip as ox


def _idx_images(pixels: np.ndarray, rows=28, cols=28, magic=2051) -> bytes:
    return struct.pack(">IIII", magic, len(pixels), rows, cols) + pixels.astype(np.uint8).tobytes()


def _idx_labels(labels, magic=2049) -> bytes:
    return struct.pack(">II", magic, len(labels)) + bytes(bytearray(labels))


def test_reference_parses_and_batches_idx_data():
    """mnist.rs:205-226: two images (zeros, 255s), labels [3, 7], one batch of 2."""
    images = np.concatenate([np.zeros((1, 784)), np.full((1, 784), 255)]).astype(np.uint8)
    assert D.parse_images(_idx_images(images)) == 2
    assert D.parse_labels(_idx_labels([3, 7])) == 2
    batches = D.MnistBatches(images, np.array([3, 7], np.uint8), 2, False)
    batch, targets = next(batches)
    assert batch.shape == (2, 1, 28, 28)
    assert targets.tolist() == [3.0, 7.0]
    np.testing.assert_array_equal(batch[0].ravel(), oracle.mnist_normalize(images[0]))
    np.testing.assert_array_equal(batch[1].ravel(), oracle.mnist_normalize(images[1]))
    with pytest.raises(StopIteration):
        next(batches)


def test_oracle_normalization_pinned_by_ieee_float32():
    """Every byte's normalized value equals numpy's float32 evaluation of
    (p / 255 - 0.1307) / 0.3081 (an independent IEEE implementation of the same operations:
    a contracted or reordered oracle would differ on some byte)."""
    p = np.arange(256, dtype=np.uint8)
    f = np.float32
    ref = (p.astype(np.float32) / f(255.0) - f(0.1307)) / f(0.3081)
    np.testing.assert_array_equal(oracle.mnist_normalize(p), ref)
    # the library's host batches equal the oracle on random images
    r = np.random.default_rng(1)
    imgs = r.integers(0, 256, (7, 784)).astype(np.uint8)
    lbls = r.integers(0, 10, 7).astype(np.uint8)
    batch, labels = D.host_batch(imgs, lbls, np.array([6, 0, 3], np.uint64))
    np.testing.assert_array_equal(batch.reshape(3, 784), oracle.mnist_normalize(imgs[[6, 0, 3]]))
    assert labels.tolist() == [float(lbls[6]), float(lbls[0]), float(lbls[3])]


@pytest.mark.parametrize("bad,message", [
    (lambda: struct.pack(">III", 2051, 1, 28), "invalid MNIST image IDX header"),
    (lambda: _idx_images(np.zeros((1, 784)), magic=2049), "invalid MNIST image IDX header"),
    (lambda: _idx_images(np.zeros((1, 27 * 28)), rows=27), "expected 28x28 MNIST images, got 27x28"),
    (lambda: _idx_images(np.zeros((2, 784)))[:-1], "invalid MNIST image payload length"),
])
def test_image_header_errors(bad, message):
    with pytest.raises(ox.OxideError) as e:
        D.parse_images(bad())
    assert e.value.status == ox.EXECUTION and message in str(e.value)


@pytest.mark.parametrize("bad,message", [
    (lambda: b"\x00\x00\x08", "invalid MNIST label IDX header"),
    (lambda: _idx_labels([1, 2], magic=2051), "invalid MNIST label IDX header"),
    (lambda: _idx_labels([1, 10]), "invalid MNIST label payload"),
    (lambda: _idx_labels([1, 2])[:-1], "invalid MNIST label payload"),
])
def test_label_header_errors(bad, message):
    with pytest.raises(ox.OxideError) as e:
        D.parse_labels(bad())
    assert e.value.status == ox.EXECUTION and message in str(e.value)


def _write_dataset(tmp_path, n_train=5, n_test=3, n_test_labels=None):
    r = np.random.default_rng(2)
    tr = r.integers(0, 256, (n_train, 784)).astype(np.uint8)
    te = r.integers(0, 256, (n_test, 784)).astype(np.uint8)
    trl = r.integers(0, 10, n_train).tolist()
    tel = r.integers(0, 10, n_test if n_test_labels is None else n_test_labels).tolist()
    (tmp_path / "train-images-idx3-ubyte").write_bytes(_idx_images(tr))
    (tmp_path / "train-labels-idx1-ubyte").write_bytes(_idx_labels(trl))
    (tmp_path / "t10k-images-idx3-ubyte").write_bytes(_idx_images(te))
    (tmp_path / "t10k-labels-idx1-ubyte").write_bytes(_idx_labels(tel))
    return tr, trl, te, tel


def test_mnist_load_and_batches(tmp_path):
    tr, trl, te, tel = _write_dataset(tmp_path)
    m = D.Mnist.load(tmp_path)
    assert (m.train_len(), m.test_len()) == (5, 3)
    np.testing.assert_array_equal(m.train_images, tr)
    # shuffled training batches: sizes 2, 2, 1 in the deterministic order
    order = oracle.mnist_order(5, True)
    got = list(m.train_batches(2, True))
    assert [b.shape[0] for b, _ in got] == [2, 2, 1]
    flat = np.concatenate([b.reshape(-1, 784) for b, _ in got])
    np.testing.assert_array_equal(flat, oracle.mnist_normalize(tr[order]))
    assert np.concatenate([lb for _, lb in got]).tolist() == [float(trl[i]) for i in order]
    # test batches keep dataset order
    tb = list(m.test_batches(16))
    assert len(tb) == 1 and tb[0][1].tolist() == [float(v) for v in tel]
    with pytest.raises(ox.OxideError) as e:
        m.train_batches(0, False)
    assert e.value.status == ox.INVALID_SHAPE


def test_mnist_load_errors(tmp_path):
    with pytest.raises(ox.OxideError) as e:
        D.Mnist.load(tmp_path / "missing")
    assert e.value.status == ox.EXECUTION and "failed to read MNIST file" in str(e.value)
    _write_dataset(tmp_path, n_test_labels=2)
    with pytest.raises(ox.OxideError) as e:
        D.Mnist.load(tmp_path)
    assert "MNIST image and label counts do not match" in str(e.value)


@pytest.mark.parametrize("count", [0, 1, 2, 3, 10, 1000, 60000])
def test_batch_order_matches_oracle(count):
    """deterministic_shuffle (mnist.rs:191-199): the library's order equals the oracle's, is a
    permutation, and is the identity without shuffling.  The concrete order is parity
    unpinned beyond the restatement (no reference output holds one)."""
    got = D.batch_order(count, True)
    np.testing.assert_array_equal(got, oracle.mnist_order(count, True))
    np.testing.assert_array_equal(np.sort(got), np.arange(count))
    np.testing.assert_array_equal(D.batch_order(count, False), np.arange(count))
    if count >= 1000:  # a shuffle, not a near-identity
        assert (got == np.arange(count)).mean() < 0.01


# ---------------------------------------------------------------- OXTR checkpoints

def test_checkpoint_bytes_match_format(tmp_path):
    tensors = [((2, 3), np.arange(6, dtype=np.float32) - 2.5), ((), np.zeros(0, np.float32)),
               ((4,), np.array([np.inf, -0.0, 1e-40, np.float32(3.4e38)], np.float32))]
    path = tmp_path / "a.oxtr"
    ox.checkpoint_save(path, tensors)
    assert path.read_bytes() == oracle.oxtr_bytes(tensors)
    # a hand-assembled golden file: magic, count 1, rank 1, dim 2, len 2, 1.0, -2.0
    gold = (b"OXTR\x01" + (1).to_bytes(8, "little") + (1).to_bytes(8, "little") +
            (2).to_bytes(8, "little") + (2).to_bytes(8, "little") +
            bytes.fromhex("0000803f") + bytes.fromhex("000000c0"))
    assert oracle.oxtr_bytes([((2,), np.array([1.0, -2.0], np.float32))]) == gold
    back = ox.checkpoint_load(path)
    assert [s for s, _ in back] == [(2, 3), (), (4,)]
    for (_, a), (_, b) in zip(back, tensors):
        np.testing.assert_array_equal(a, b.ravel())


def test_checkpoint_read_errors(tmp_path):
    def load(b):
        p = tmp_path / "x.oxtr"
        p.write_bytes(b)
        with pytest.raises(ox.OxideError) as e:
            ox.checkpoint_load(p)
        assert e.value.status == ox.EXECUTION
        return str(e.value)

    assert "failed to open checkpoint" in str(pytest.raises(
        ox.OxideError, ox.checkpoint_load, tmp_path / "none.oxtr").value)
    assert "invalid OXTR checkpoint header" in load(b"OXTR\x02" + bytes(8))
    good = oracle.oxtr_bytes([((3,), np.ones(3, np.float32))])
    load(good[:-1])                                          # truncated values
    load(good[:9])                                           # truncated count
    load(b"OXTR\x01" + (2 ** 62).to_bytes(8, "little"))      # absurd count, no data
    load(b"OXTR\x01" + (1).to_bytes(8, "little") + (2 ** 61).to_bytes(8, "little"))
