"""GPU parity of fdl_idx_gather, the IDX batch gather (byte rows in HBM ->
fp32 rows / 255 and int64 labels).

Integer and byte work, so every comparison is bit-exact: against the oracle's
restatement of legacy/src/data/DataLoader.cpp:61-68,87-90, and for the pixel
conversion against the correctly rounded quotients found from exact
rationals.  Cases cover the 4-pixel vector path and the byte path (odd row
lengths, misaligned pointers), each with normal and streaming stores (outputs
of 32 MiB and more), out-of-range and duplicate indices, empty inputs,
labels-only and pixels-only calls, and the full MNIST-sized set.
"""
import numpy as np
import pytest

import fast_dl_amd.capi as capi
import oracle
from tests import idx_files
from tests.conftest import rng
from tests.gpu_helpers import dev, host, say, stream

pytestmark = pytest.mark.gpu


def _gather(images, labels, index, batch, divisor=255.0, want_x=True, want_y=True,
            img_offset=0, x_offset=0):
    """Run fdl_idx_gather; img_offset / x_offset (bytes / floats) misalign the
    device pointers to force the byte path.  Returns host (x, y)."""
    import torch

    count, row_bytes = images.shape
    buf = torch.zeros(images.size + img_offset + 16, dtype=torch.uint8, device="cuda")
    if images.size:
        buf[img_offset:img_offset + images.size] = dev(images.reshape(-1))
    dlab = dev(labels) if labels is not None and labels.size else None
    didx = dev(index) if index is not None and index.size else None
    xbuf = torch.full((batch * row_bytes + x_offset + 4,), float("nan"), device="cuda")
    y = torch.full((max(batch, 1),), 12345, dtype=torch.int64, device="cuda")
    capi.idx_gather(buf.data_ptr() + img_offset, dlab.data_ptr() if dlab is not None else None,
                    count, row_bytes, didx.data_ptr() if didx is not None else None, batch,
                    divisor, xbuf.data_ptr() + 4 * x_offset if want_x else None,
                    y.data_ptr() if want_y else None, stream())
    x = host(xbuf)[x_offset:x_offset + batch * row_bytes].reshape(batch, row_bytes)
    return x, host(y)[:batch]


def _expect(images, labels, index, batch, divisor=255.0):
    return oracle.idx_gather(images, labels, index, batch=batch, divisor=divisor)


def test_every_byte_value_is_correctly_rounded(device):
    images = np.arange(256, dtype=np.uint8).reshape(1, 256)
    say("idx_gather: all 256 byte values, vector path")
    x, _ = _gather(images, None, None, 1, want_y=False)
    q = idx_files.correctly_rounded_quotients(255)
    assert np.array_equal(x[0].view(np.uint32), q.view(np.uint32))
    # one byte per row: the byte path, and every label byte through int8
    rows = np.arange(256, dtype=np.uint8).reshape(256, 1)
    say("idx_gather: all 256 byte values, byte path with labels")
    x, y = _gather(rows, rows[:, 0].copy(), None, 256)
    assert np.array_equal(x[:, 0].view(np.uint32), q.view(np.uint32))
    assert np.array_equal(y, np.arange(256, dtype=np.uint8).astype(np.int8).astype(np.int64))


CASES = [
    # (count, row_bytes, batch, index kind, divisor, img_offset, x_offset)
    (100, 784, 100, None, 255.0, 0, 0),
    (1000, 784, 256, "perm", 255.0, 0, 0),
    (37, 5, 50, "oob", 255.0, 0, 0),
    (64, 3, 200, "dup", 255.0, 0, 0),
    (10, 4, 3, "perm", 255.0, 0, 0),
    (300, 1000, 333, "oob", 7.5, 0, 0),
    (5, 1, 7, "oob", -3.0, 0, 0),
    (200, 784, 129, "perm", 255.0, 1, 0),   # misaligned images: byte path
    (200, 784, 129, "perm", 255.0, 0, 1),   # x not 16-byte aligned: byte path
    (3000, 12, 2999, None, 1.0, 0, 0),
    # outputs of 32 MiB and more take streaming stores
    (11000, 784, 11000, "oob", 255.0, 0, 0),
    (12000, 785, 12000, "perm", 255.0, 0, 0),
]


@pytest.mark.parametrize("count,row_bytes,batch,kind,divisor,img_offset,x_offset", CASES)
def test_gather_matches_oracle(device, count, row_bytes, batch, kind, divisor, img_offset,
                               x_offset):
    g = rng(40 + count + row_bytes + batch)
    images = g.integers(0, 256, (count, row_bytes), dtype=np.uint8)
    labels = g.integers(0, 256, count, dtype=np.uint8)
    if kind is None:
        index = None
    elif kind == "perm":
        index = g.permutation(count)[:batch].astype(np.int64)
    elif kind == "dup":
        index = g.integers(0, count, batch).astype(np.int64)
    else:  # out of range entries mixed in
        index = g.integers(0, count, batch).astype(np.int64)
        index[::7] = -1
        index[3::11] = count
        index[5::13] = 1 << 40
        index[6::17] = -(1 << 62)
    say(f"idx_gather count={count} row_bytes={row_bytes} batch={batch} index={kind} "
        f"divisor={divisor} offsets={img_offset},{x_offset}")
    x, y = _gather(images, labels, index, batch, divisor, img_offset=img_offset,
                   x_offset=x_offset)
    ex, ey = _expect(images, labels, index, batch, divisor)
    assert np.array_equal(x.view(np.uint32), ex.view(np.uint32))
    assert np.array_equal(y, ey)


def test_labels_only_pixels_only_and_empty(device):
    g = rng(50)
    images = g.integers(0, 256, (20, 784), dtype=np.uint8)
    labels = g.integers(0, 10, 20, dtype=np.uint8)
    index = np.array([19, 0, 5, 5, 25], np.int64)
    ex, ey = _expect(images, labels, index, 5)
    say("idx_gather labels only")
    _, y = _gather(images, labels, index, 5, want_x=False)
    assert np.array_equal(y, ey)
    say("idx_gather pixels only")
    x, y = _gather(images, labels, index, 5, want_y=False)
    assert np.array_equal(x, ex)
    assert np.all(y == 12345)  # y untouched
    say("idx_gather count 0: every row out of range")
    x, y = _gather(np.zeros((0, 784), np.uint8), np.zeros(0, np.uint8), index, 5)
    assert np.all(x == 0) and np.all(y == -1)
    say("idx_gather batch 0")
    x, y = _gather(images, labels, np.zeros(0, np.int64), 0)
    assert x.size == 0 and y.size == 0


def test_real_labels_and_full_mnist_sized_set(device):
    # The reference's MNIST label file with synthetic 28x28 images (the image
    # files are not in the reference snapshot); the whole set in one launch.
    labels = np.frombuffer(open(idx_files.TRAIN_LABELS, "rb").read()[8:], np.uint8).copy()
    count = labels.size
    g = rng(51)
    images = g.integers(0, 256, (count, 784), dtype=np.uint8)
    say("idx_gather whole 60000x784 set, no index")
    x, y = _gather(images, labels, None, count)
    assert np.array_equal(x, images.astype(np.float32) / np.float32(255))
    assert np.array_equal(y, oracle.idx_read_labels(idx_files.TRAIN_LABELS))
    assert np.bincount(y).tolist() == idx_files.MNIST_TRAIN_CLASS_COUNTS
    perm = g.permutation(count).astype(np.int64)
    say("idx_gather 60000 rows in a permuted order")
    xp, yp = _gather(images, labels, perm, count)
    assert np.array_equal(xp, x[perm])
    assert np.array_equal(yp, y[perm])
