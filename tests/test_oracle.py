"""Pins the CPU oracle (oracle/) before any GPU result is compared with it.

Each check is independent of the oracle's own text: the reference's fixtures
(quoted with file:line), fp64 numpy, closed forms, transposition and batching
identities, exact integer arithmetic and finite differences.  The last test
plants plausible mistakes in the oracle's inputs/outputs on the CPU and shows
that these same checks reject them.
"""
import numpy as np
import pytest

import oracle
from tests.conftest import rng

# ---------------------------------------------------------------------------
# Reference fixtures
# ---------------------------------------------------------------------------

# tests/tensor/matmul_tensor_test.cpp:30-42 (A 2x3, B 3x4); expected values are
# the products worked by hand: row0 = [1,2,3].B, row1 = [4,5,6].B.
MATMUL_A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
MATMUL_B = np.array([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]], np.float32)
MATMUL_C = np.array([[38, 44, 50, 56], [83, 98, 113, 128]], np.float32)

# tests/tensor/linear_tensor_test.cpp:38-53 (W is [in=3, out=2]).
LINEAR_X = MATMUL_A
LINEAR_W = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
LINEAR_B = np.array([0.5, 1.0], np.float32)
LINEAR_Y = np.array([[22.5, 29.0], [49.5, 65.0]], np.float32)

# tests/nn/relu_module_test.cpp:22-29
RELU_IN = np.array([-2.0, -0.5, 0.0, 1.5, 3.0, -4.0], np.float32)
RELU_OUT = np.array([0.0, 0.0, 0.0, 1.5, 3.0, 0.0], np.float32)

# tests/tensor/cross_entropy_tensor_test.cpp:40-44; 0.4076059 = log(1 + e^-1 + e^-2)
CE_LOGITS = np.array([[1, 2, 3], [1, 3, 2]], np.float32)
CE_LABELS = np.array([2, 1], np.int64)
CE_LOSS = 0.4076059

# tests/tensor/softmax_tensor_test.cpp:43-46
SOFTMAX_IN = np.array([[1, 2, 3, 4], [1, 3, 2, 0]], np.float32)


def close_abs(a, b, tol):
    return bool(np.all(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)) <= tol))


def test_matmul_fixture():
    assert np.array_equal(oracle.gemm_cpu(MATMUL_A, MATMUL_B), MATMUL_C)
    c = oracle.sgemm_ex(0, 0, MATMUL_A, MATMUL_B, 2, 4, 3)[0]
    assert np.array_equal(c, MATMUL_C)


def test_linear_fixture():
    assert close_abs(oracle.linear(LINEAR_X, LINEAR_W, LINEAR_B), LINEAR_Y, 1e-4)
    y = oracle.sgemm_ex(0, 0, LINEAR_X, LINEAR_W, 2, 2, 3, bias=LINEAR_B,
                        epilogue=oracle.EPI_BIAS)[0]
    assert close_abs(y, LINEAR_Y, 1e-4)


def test_relu_fixture():
    assert np.array_equal(oracle.relu(RELU_IN), RELU_OUT)


def test_cross_entropy_fixture_and_closed_forms():
    assert abs(oracle.cross_entropy(CE_LOGITS, CE_LABELS) - CE_LOSS) < 1e-6
    assert abs(CE_LOSS - np.log(1 + np.exp(-1) + np.exp(-2))) < 1e-6
    # Uniform logits: loss = log(C) for any label.
    z = np.full((5, 7), 0.3, np.float32)
    assert abs(oracle.cross_entropy(z, np.arange(5)) - np.log(7)) < 1e-6
    # Invalid labels add nothing but still count in the batch
    # (src/kernels/cuda/cross_entropy.cu:16-19,34).
    lab = np.array([2, -1], np.int64)
    assert abs(oracle.cross_entropy(CE_LOGITS, lab) - CE_LOSS / 2) < 1e-6


def test_softmax_fixture():
    y = oracle.softmax(SOFTMAX_IN)
    x = SOFTMAX_IN.astype(np.float64)
    ref = np.exp(x - x.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert close_abs(y, ref, 1e-6)
    assert close_abs(y.sum(1), 1.0, 1e-6)
    assert close_abs(oracle.softmax(SOFTMAX_IN + 100.0), y, 1e-6)  # shift invariance


# ---------------------------------------------------------------------------
# GEMM against fp64, identities, exact arithmetic
# ---------------------------------------------------------------------------

def gemm_within_tolerance(c32, c64, abs_ab, K) -> bool:
    tol = oracle.gemm_tolerance(abs_ab, K)
    return bool(np.all(np.abs(c32.astype(np.float64) - c64) <= tol))


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 5, 3), (33, 17, 65), (64, 48, 300)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_ex_matches_fp64(M, N, K, ta, tb):
    g = rng(M * 1000 + N * 10 + K)
    A = g.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = g.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    c32 = oracle.sgemm_ex(ta, tb, A, B, M, N, K)[0]
    opA = A.T if ta else A
    opB = B.T if tb else B
    c64 = opA.astype(np.float64) @ opB.astype(np.float64)
    abs_ab = np.abs(opA).astype(np.float64) @ np.abs(opB).astype(np.float64)
    assert gemm_within_tolerance(c32, c64, abs_ab, K)
    c64o, s64o = oracle.sgemm_ex_f64(ta, tb, A, B, M, N, K)
    assert np.allclose(c64o[0], c64, rtol=1e-12, atol=1e-12)
    assert np.allclose(s64o[0], abs_ab, rtol=1e-12, atol=1e-12)


def test_transpose_identities_bit_exact():
    g = rng(7)
    M, N, K = 19, 23, 31
    A = g.standard_normal((M, K)).astype(np.float32)
    B = g.standard_normal((K, N)).astype(np.float32)
    nn = oracle.sgemm_ex(0, 0, A, B, M, N, K)
    assert np.array_equal(oracle.sgemm_ex(1, 0, np.ascontiguousarray(A.T), B, M, N, K), nn)
    assert np.array_equal(oracle.sgemm_ex(0, 1, A, np.ascontiguousarray(B.T), M, N, K), nn)
    assert np.array_equal(
        oracle.sgemm_ex(1, 1, np.ascontiguousarray(A.T), np.ascontiguousarray(B.T), M, N, K), nn)
    # The restated gemm_cpu is the NN case.
    assert np.array_equal(oracle.gemm_cpu(A, B), nn[0])


def test_batched_equals_loop():
    g = rng(11)
    batch, M, N, K = 5, 9, 13, 17
    A = g.standard_normal((batch, M, K)).astype(np.float32)
    B = g.standard_normal((batch, N, K)).astype(np.float32)
    c = oracle.sgemm_ex(0, 1, A, B, M, N, K, batch=batch)
    for i in range(batch):
        assert np.array_equal(c[i], oracle.sgemm_ex(0, 1, A[i], B[i], M, N, K)[0])


def test_integer_inputs_exact():
    g = rng(3)
    M, N, K = 40, 30, 200
    A = g.integers(-8, 9, (M, K)).astype(np.float32)
    B = g.integers(-8, 9, (K, N)).astype(np.float32)
    exact = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(oracle.gemm_cpu(A, B), exact.astype(np.float32))


def test_epilogues_closed_form():
    g = rng(5)
    M, N, K = 12, 10, 8
    A = g.standard_normal((M, K)).astype(np.float32)
    B = g.standard_normal((K, N)).astype(np.float32)
    bias = g.standard_normal(N).astype(np.float32)
    plain = oracle.sgemm_ex(0, 0, A, B, M, N, K)[0]
    with_b = oracle.sgemm_ex(0, 0, A, B, M, N, K, bias=bias, epilogue=oracle.EPI_BIAS)[0]
    assert np.array_equal(with_b, plain + bias)  # bias added after the whole sum
    br = oracle.sgemm_ex(0, 0, A, B, M, N, K, bias=bias, epilogue=oracle.EPI_BIAS_RELU)[0]
    assert np.array_equal(br, np.maximum(plain + bias, 0))
    r = oracle.sgemm_ex(0, 0, A, B, M, N, K, epilogue=oracle.EPI_RELU)[0]
    assert np.array_equal(r, np.maximum(plain, 0))
    aux = g.standard_normal((M, N)).astype(np.float32)
    rg = oracle.sgemm_ex(0, 0, A, B, M, N, K, aux=aux, epilogue=oracle.EPI_RELU_GRAD)[0]
    assert np.array_equal(rg, np.where(aux > 0, plain, 0))


def test_colsum_relu_backward_sgd():
    g = rng(9)
    x = g.standard_normal((37, 11)).astype(np.float32)
    assert close_abs(oracle.colsum(x), x.astype(np.float64).sum(0), 1e-5)
    act = g.standard_normal((37, 11)).astype(np.float32)
    assert np.array_equal(oracle.relu_backward(x, act), np.where(act > 0, x, 0))
    p = g.standard_normal(50).astype(np.float32)
    d = g.standard_normal(50).astype(np.float32)
    assert np.array_equal(oracle.sgd(p, d, 0.1), p - np.float32(0.1) * d)


# ---------------------------------------------------------------------------
# Gradients: finite differences
# ---------------------------------------------------------------------------

def ce_loss_f64(z, labels):
    z = z.astype(np.float64)
    m = z.max(1, keepdims=True)
    lse = np.log(np.exp(z - m).sum(1)) + m[:, 0]
    valid = (labels >= 0) & (labels < z.shape[1])
    pick = z[np.arange(len(labels)), np.where(valid, labels, 0)]
    return float(np.sum(np.where(valid, lse - pick, 0.0)) / len(labels))


def test_softmax_xent_grad_finite_differences():
    g = rng(13)
    z = g.standard_normal((6, 5)).astype(np.float32)
    labels = np.array([0, 4, 2, 2, -1, 1], np.int64)
    grad = oracle.softmax_xent_grad(z, labels)
    h = 1e-6
    num = np.zeros_like(z, dtype=np.float64)
    for i in range(z.shape[0]):
        for j in range(z.shape[1]):
            zp = z.astype(np.float64).copy()
            zm = zp.copy()
            zp[i, j] += h
            zm[i, j] -= h
            num[i, j] = (ce_loss_f64(zp, labels) - ce_loss_f64(zm, labels)) / (2 * h)
    valid = labels >= 0
    assert np.max(np.abs(grad[valid] - num[valid])) < 1e-6
    # rows with a valid label sum to zero
    assert np.all(np.abs(grad[valid].sum(1)) < 1e-7)
    # An invalid-label row keeps p / batch (legacy SoftmaxCrossEntropyLoss.cpp:43-50
    # subtracts the one-hot only for valid labels), although the loss ignores it.
    p = np.exp(z[~valid].astype(np.float64) - z[~valid].max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.max(np.abs(grad[~valid] - p / len(labels))) < 1e-7


def mlp_case(seed, B=3, I=6, H=5, C=4):
    g = rng(seed)
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = (g.standard_normal((I, H)) * 0.7).astype(np.float32)
    b1 = (g.standard_normal(H) * 0.1).astype(np.float32)
    W2 = (g.standard_normal((H, C)) * 0.7).astype(np.float32)
    b2 = (g.standard_normal(C) * 0.1).astype(np.float32)
    return X, labels, W1, b1, W2, b2


def test_mlp_grads_f64_finite_differences():
    X, labels, W1, b1, W2, b2 = mlp_case(21)
    params = [p.astype(np.float64) for p in (W1, b1, W2, b2)]
    Xd = X.astype(np.float64)
    grads = oracle.mlp2_grads_f64(Xd, labels, *params)
    h = 1e-6

    def loss(ps, x=Xd):
        return oracle.mlp2_loss_f64(x, labels, *ps)

    for idx, name in enumerate(["dW1", "db1", "dW2", "db2"]):
        p = params[idx]
        num = np.zeros_like(p)
        for flat in range(p.size):
            pp = [q.copy() for q in params]
            pm = [q.copy() for q in params]
            pp[idx].reshape(-1)[flat] += h
            pm[idx].reshape(-1)[flat] -= h
            num.reshape(-1)[flat] = (loss(pp) - loss(pm)) / (2 * h)
        assert np.max(np.abs(grads[name] - num)) < 1e-7, name
    numx = np.zeros_like(Xd)
    for flat in range(Xd.size):
        xp = Xd.copy()
        xm = Xd.copy()
        xp.reshape(-1)[flat] += h
        xm.reshape(-1)[flat] -= h
        numx.reshape(-1)[flat] = (loss(params, xp) - loss(params, xm)) / (2 * h)
    assert np.max(np.abs(grads["dX"] - numx)) < 1e-7


def test_mlp_step_fp32_matches_fp64_and_sgd():
    X, labels, W1, b1, W2, b2 = mlp_case(22, B=8, I=20, H=16, C=10)
    lr = 0.05
    out = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, lr)
    ref = oracle.mlp2_grads_f64(X, labels, W1, b1, W2, b2)
    for name in ("dW1", "db1", "dW2", "db2", "dX"):
        assert np.max(np.abs(out[name] - ref[name])) < 1e-5, name
    assert abs(out["loss"][0] - oracle.mlp2_loss_f64(X, labels, W1, b1, W2, b2)) < 1e-5
    assert np.array_equal(out["W1"], W1 - np.float32(lr) * out["dW1"])
    assert np.array_equal(out["b2"], b2 - np.float32(lr) * out["db2"])


# ---------------------------------------------------------------------------
# The checks above reject plausible mistakes (planted on the CPU only)
# ---------------------------------------------------------------------------

def test_checks_catch_planted_mistakes():
    # transposed operand: the non-square fixture no longer matches
    wrong = oracle.sgemm_ex(0, 1, MATMUL_A, MATMUL_B[:, :3].copy(), 2, 3, 3)[0]
    assert not np.array_equal(wrong, MATMUL_C[:, :3])
    # dropped last k term
    short = oracle.gemm_cpu(MATMUL_A[:, :2].copy(), MATMUL_B[:2].copy())
    assert not np.array_equal(short, MATMUL_C)
    # bias on the wrong axis (per row instead of per column)
    y = oracle.sgemm_ex(0, 0, LINEAR_X, LINEAR_W, 2, 2, 3)[0] + LINEAR_B[:, None]
    assert not close_abs(y, LINEAR_Y, 1e-4)
    # wrong index in a random GEMM fails the fp64 tolerance check
    g = rng(1)
    M, N, K = 16, 16, 64
    A = g.standard_normal((M, K)).astype(np.float32)
    B = g.standard_normal((K, N)).astype(np.float32)
    c64 = A.astype(np.float64) @ B.astype(np.float64)
    s64 = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    good = oracle.sgemm_ex(0, 0, A, B, M, N, K)[0]
    assert gemm_within_tolerance(good, c64, s64, K)
    assert not gemm_within_tolerance(oracle.sgemm_ex(1, 0, A[:, :M].copy(), B[:M].copy(),
                                                     M, N, M)[0], c64, s64, K)
    assert not gemm_within_tolerance(good[::-1].copy(), c64, s64, K)
    # sign flip in the CE gradient fails the finite-difference check
    z = g.standard_normal((3, 4)).astype(np.float32)
    lab = np.array([1, 0, 3], np.int64)
    grad = oracle.softmax_xent_grad(z, lab)
    h = 1e-6
    zp = z.astype(np.float64).copy()
    zm = zp.copy()
    zp[0, 1] += h
    zm[0, 1] -= h
    num = (ce_loss_f64(zp, lab) - ce_loss_f64(zm, lab)) / (2 * h)
    assert abs(grad[0, 1] - num) < 1e-6
    assert abs(-grad[0, 1] - num) > 1e-3


# ---------------------------------------------------------------------------
# IDX files (legacy/src/data/DataLoader.cpp)
# ---------------------------------------------------------------------------

from tests import idx_files  # noqa: E402


def test_idx_labels_match_published_mnist_facts():
    # The reference's own label files (mnist/*-labels-idx1-ubyte, shipped as
    # tests/golden/mnist fixtures) against published MNIST figures.
    for path, counts, first in [
            (idx_files.TRAIN_LABELS, idx_files.MNIST_TRAIN_CLASS_COUNTS, idx_files.MNIST_TRAIN_FIRST),
            (idx_files.TEST_LABELS, idx_files.MNIST_TEST_CLASS_COUNTS, idx_files.MNIST_TEST_FIRST)]:
        lab = oracle.idx_read_labels(path)
        assert lab.size == sum(counts)
        assert np.bincount(lab, minlength=10).tolist() == counts
        assert lab[:10].tolist() == first
        # the num limit keeps the first records (DataLoader.cpp:85)
        assert oracle.idx_read_labels(path, num=7).tolist() == first[:7]
        assert oracle.idx_read_labels(path, num=10 ** 6).size == lab.size


def test_idx_images_synthetic_file(tmp_path):
    g = rng(30)
    # rows != cols and a count of 0x102 make a byte-order slip visible
    imgs = g.integers(0, 256, (258, 3, 5), dtype=np.uint8)
    path = str(tmp_path / "img")
    idx_files.write_idx3(path, imgs)
    assert oracle.idx_image_dims(path) == (258, 3, 5)
    x = oracle.idx_read_images(path)
    assert x.shape == (258, 15)
    assert np.array_equal(x, imgs.reshape(258, 15).astype(np.float32) / np.float32(255))
    assert np.array_equal(oracle.idx_read_images(path, num=4), x[:4])
    assert oracle.idx_image_dims(path, num=300) == (258, 3, 5)


def test_idx_pixel_conversion_is_correctly_rounded(tmp_path):
    imgs = np.arange(256, dtype=np.uint8).reshape(1, 16, 16)
    path = str(tmp_path / "all_bytes")
    idx_files.write_idx3(path, imgs)
    x = oracle.idx_read_images(path)[0]
    assert np.array_equal(x.view(np.uint32), idx_files.correctly_rounded_quotients(255).view(np.uint32))
    assert x[0] == 0.0 and x[255] == 1.0


def test_idx_label_bytes_read_through_signed_char(tmp_path):
    path = str(tmp_path / "lab")
    idx_files.write_idx1(path, np.array([0, 9, 127, 128, 200, 255], np.uint8))
    assert oracle.idx_read_labels(path).tolist() == [0, 9, 127, -128, -56, -1]


def test_idx_rejects_bad_files(tmp_path):
    imgs = np.zeros((4, 2, 2), np.uint8)
    cases = [("magic", dict(magic=0x801), -2), ("short", dict(truncate=1), -3),
             ("header", dict(truncate=4 * 4 + 1), -3), ("neg", dict(count=-5), -4)]
    for name, kw, code in cases:
        path = str(tmp_path / name)
        idx_files.write_idx3(path, imgs, **kw)
        with pytest.raises(oracle.IdxError) as e:
            oracle.idx_read_images(path)
        assert e.value.code == code, name
    with pytest.raises(oracle.IdxError) as e:
        oracle.idx_read_images(str(tmp_path / "missing"))
    assert e.value.code == -1
    path = str(tmp_path / "lab")
    idx_files.write_idx1(path, np.arange(5, dtype=np.uint8), magic=0x803)
    with pytest.raises(oracle.IdxError) as e:
        oracle.idx_read_labels(path)
    assert e.value.code == -2
    idx_files.write_idx1(path, np.arange(5, dtype=np.uint8), truncate=1)
    with pytest.raises(oracle.IdxError) as e:
        oracle.idx_read_labels(path)
    assert e.value.code == -3


def test_idx_gather_equals_indexing():
    g = rng(31)
    images = g.integers(0, 256, (50, 13), dtype=np.uint8)
    labels = g.integers(0, 256, 50, dtype=np.uint8)
    index = np.array([3, 3, 49, 0, -1, 50, 17, 1 << 40], np.int64)
    x, y = oracle.idx_gather(images, labels, index)
    full = images.astype(np.float32) / np.float32(255)
    ok = (index >= 0) & (index < 50)
    assert np.array_equal(x[ok], full[index[ok]])
    assert np.all(x[~ok] == 0)
    assert np.array_equal(y[ok], labels[index[ok]].astype(np.int8).astype(np.int64))
    assert np.all(y[~ok] == -1)
    x2, _ = oracle.idx_gather(images, None, None, batch=50, divisor=3.0)
    assert np.array_equal(x2, images.astype(np.float32) / np.float32(3))


def test_idx_checks_catch_planted_mistakes(tmp_path):
    import struct
    raw = open(idx_files.TRAIN_LABELS, "rb").read()
    # little-endian header words: wrong magic and count
    magic, count = struct.unpack("<ii", raw[:8])
    assert magic != 0x801 and count != 60000
    # labels read as unsigned bytes: the signed-char case fails
    assert (np.array([128, 200], np.uint8).astype(np.int64) != [-128, -56]).all()
    # multiplying by 1/255 instead of dividing: not correctly rounded
    b = np.arange(256, dtype=np.float32)
    assert not np.array_equal(b * (np.float32(1) / np.float32(255)),
                              idx_files.correctly_rounded_quotients(255))
    # an off-by-one row in the gather fails the indexing identity
    g = rng(32)
    images = g.integers(0, 256, (8, 4), dtype=np.uint8)
    x, _ = oracle.idx_gather(images, None, np.array([2, 5], np.int64))
    assert not np.array_equal(x, images[[3, 6]].astype(np.float32) / np.float32(255))
