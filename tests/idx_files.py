"""Writers of IDX (MNIST) files for the loader tests, from the published
format: a big-endian 32-bit magic (0x00000803 for images, 0x00000801 for
labels), big-endian 32-bit dimensions (count, then rows and cols for
images), then one unsigned byte per element, row-major."""
from __future__ import annotations

import os
import struct

import numpy as np

GOLDEN_MNIST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mnist")
TRAIN_LABELS = os.path.join(GOLDEN_MNIST, "train-labels-idx1-ubyte")
TEST_LABELS = os.path.join(GOLDEN_MNIST, "t10k-labels-idx1-ubyte")

# Published facts about the MNIST label files (LeCun et al.): record counts,
# images per class 0..9, and the first ten labels of each file.
MNIST_TRAIN_CLASS_COUNTS = [5923, 6742, 5958, 6131, 5842, 5421, 5918, 6265, 5851, 5949]
MNIST_TEST_CLASS_COUNTS = [980, 1135, 1032, 1010, 982, 892, 958, 1028, 974, 1009]
MNIST_TRAIN_FIRST = [5, 0, 4, 1, 9, 2, 1, 3, 1, 4]
MNIST_TEST_FIRST = [7, 2, 1, 0, 4, 1, 4, 9, 5, 9]


def write_idx3(path: str, images: np.ndarray, magic: int = 0x803, count: int | None = None,
               truncate: int = 0) -> None:
    images = np.ascontiguousarray(images, dtype=np.uint8)
    n, rows, cols = images.shape
    data = struct.pack(">iiii", magic, n if count is None else count, rows, cols) + images.tobytes()
    with open(path, "wb") as f:
        f.write(data[:len(data) - truncate])


def write_idx1(path: str, labels: np.ndarray, magic: int = 0x801, count: int | None = None,
               truncate: int = 0) -> None:
    labels = np.ascontiguousarray(labels, dtype=np.uint8)
    data = struct.pack(">ii", magic, labels.size if count is None else count) + labels.tobytes()
    with open(path, "wb") as f:
        f.write(data[:len(data) - truncate])


def correctly_rounded_quotients(divisor: int = 255) -> np.ndarray:
    """float32 nearest to b / divisor for every byte b, found from exact
    rationals (ties to even), independent of any float division."""
    from fractions import Fraction

    out = np.empty(256, np.float32)
    for b in range(256):
        q = Fraction(b, divisor)
        f = np.float32(float(q))  # within one ulp of q
        cands = [np.nextafter(f, np.float32(-1)), f, np.nextafter(f, np.float32(2))]
        errs = [abs(Fraction(float(c)) - q) for c in cands]
        best = min(errs)
        ties = [c for c, e in zip(cands, errs) if e == best]
        if len(ties) > 1:  # ties to even mantissa
            ties = [c for c in ties if (int(np.float32(c).view(np.uint32)) & 1) == 0]
        out[b] = ties[0]
    return out
