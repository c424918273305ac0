"""CPU oracle for the fp32 GEMM path -- TEST INFRASTRUCTURE ONLY.

numpy front-end over ``oracle/liboracle.so`` (plain C, ``oracle/oracle.c``),
which restates the reference's own CPU loops (file:line citations in
``oracle/oracle.h``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, as the checker
or the timed CPU baseline; the product package ``fast_dl_amd`` never does.

Parity pinning of each function is listed in ``oracle/oracle.h`` and tested
in ``tests/test_oracle.py``.  Nothing here is "parity unpinned" except the
random fills, which the oracle does not restate (the reference's cuRAND
stream is closed; its tests pin only range and same-seed determinism).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

FLT_EPS = float(np.finfo(np.float32).eps)  # 2**-23

EPI_NONE, EPI_BIAS, EPI_BIAS_RELU, EPI_RELU, EPI_RELU_GRAD = range(5)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_int = ctypes.c_int
_flt = ctypes.c_float

_SIGS = {
    "oracle_gemm_cpu": (None, [_vp, _vp, _vp, _sz, _sz, _sz]),
    "oracle_gemm_cpu_rows": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz]),
    "oracle_sgemm_ex": (None, [_int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                               _vp, _i64, _i64, _i64, _vp, _vp, _int]),
    "oracle_sgemm_ex_f64": (None, [_int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                   _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _int]),
    "oracle_linear": (None, [_vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "oracle_relu": (None, [_vp, _vp, _sz]),
    "oracle_relu_backward": (None, [_vp, _vp, _vp, _sz]),
    "oracle_colsum": (None, [_vp, _vp, _sz, _sz]),
    "oracle_softmax": (None, [_vp, _vp, _sz, _sz]),
    "oracle_cross_entropy": (_flt, [_vp, _vp, _sz, _sz]),
    "oracle_softmax_xent_grad": (None, [_vp, _vp, _vp, _sz, _sz]),
    "oracle_sgd": (None, [_vp, _vp, _flt, _sz]),
    "oracle_mlp2_train_step": (None, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                      _flt, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oracle_mlp2_loss_f64": (ctypes.c_double, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp,
                                               _vp, _vp]),
    "oracle_mlp2_grads_f64": (None, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _vp, _vp]),
    "oracle_idx_read_images": (_int, [ctypes.c_char_p, _i64, _vp, _vp, _vp, _vp]),
    "oracle_idx_read_labels": (_int, [ctypes.c_char_p, _i64, _vp, _vp]),
    "oracle_idx_gather": (None, [_vp, _vp, _i64, _i64, _vp, _i64, _flt, _vp, _vp]),
}


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            subprocess.run(["make", "-C", _HERE, "-s"], check=True)
        _LIB = ctypes.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_LIB, name)
            fn.restype = res
            fn.argtypes = args
    return _LIB


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def gemm_cpu(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """gemm_benchmark.cu:14-26 on row-major a[m,k], b[k,n]."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().oracle_gemm_cpu(_p(a), _p(b), _p(c), m, n, k)
    return c


def gemm_cpu_rows(a: np.ndarray, b: np.ndarray, row0: int, row1: int) -> np.ndarray:
    """Rows [row0, row1) of gemm_cpu (returns only those rows)."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32)
    lib().oracle_gemm_cpu_rows(_p(a), _p(b), _p(c), m, n, k, row0, row1)
    return c[row0:row1]


def _ex_shapes(ta, tb, M, N, K, batch):
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    return a_rows, a_cols, b_rows, b_cols


def sgemm_ex(ta: int, tb: int, A: np.ndarray, B: np.ndarray, M: int, N: int, K: int,
             batch: int = 1, bias=None, aux=None, epilogue: int = EPI_NONE) -> np.ndarray:
    """Strided-batched fp32 GEMM on packed operands (A is [batch, *op-shape])."""
    A, B = _f32(A), _f32(B)
    a_rows, a_cols, b_rows, b_cols = _ex_shapes(ta, tb, M, N, K, batch)
    C = np.empty((batch, M, N), np.float32)
    bias = None if bias is None else _f32(bias)
    aux = None if aux is None else _f32(aux)
    lib().oracle_sgemm_ex(ta, tb, M, N, K, _p(A), max(1, a_cols), a_rows * a_cols,
                          _p(B), max(1, b_cols), b_rows * b_cols, _p(C), max(1, N), M * N,
                          batch, _p(bias), _p(aux), epilogue)
    return C


def sgemm_ex_f64(ta: int, tb: int, A: np.ndarray, B: np.ndarray, M: int, N: int, K: int,
                 batch: int = 1, bias=None, aux=None, epilogue: int = EPI_NONE):
    """fp64 twin: returns (C64, ABS64) where ABS64 = |A||B| (+|bias|) elementwise."""
    A, B = _f32(A), _f32(B)
    a_rows, a_cols, b_rows, b_cols = _ex_shapes(ta, tb, M, N, K, batch)
    C = np.empty((batch, M, N), np.float64)
    S = np.empty((batch, M, N), np.float64)
    bias = None if bias is None else _f32(bias)
    aux = None if aux is None else _f32(aux)
    lib().oracle_sgemm_ex_f64(ta, tb, M, N, K, _p(A), max(1, a_cols), a_rows * a_cols,
                              _p(B), max(1, b_cols), b_rows * b_cols, _p(C), _p(S), max(1, N),
                              M * N, batch, _p(bias), _p(aux), epilogue)
    return C, S


def linear(x, w, bias) -> np.ndarray:
    x, w, bias = _f32(x), _f32(w), _f32(bias)
    bsz, fin = x.shape
    fout = w.shape[1]
    y = np.empty((bsz, fout), np.float32)
    lib().oracle_linear(_p(x), _p(w), _p(bias), _p(y), bsz, fin, fout)
    return y


def relu(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_relu(_p(x), _p(y), x.size)
    return y


def relu_backward(g, act) -> np.ndarray:
    g, act = _f32(g), _f32(act)
    out = np.empty_like(g)
    lib().oracle_relu_backward(_p(g), _p(act), _p(out), g.size)
    return out


def colsum(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty((x.shape[1],), np.float32)
    lib().oracle_colsum(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def softmax(x) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    lib().oracle_softmax(_p(x), _p(y), x.shape[0], x.shape[1])
    return y


def cross_entropy(logits, labels) -> float:
    logits = _f32(logits)
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    return float(lib().oracle_cross_entropy(_p(logits), _p(labels), logits.shape[0],
                                            logits.shape[1]))


def softmax_xent_grad(logits, labels) -> np.ndarray:
    logits = _f32(logits)
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    g = np.empty_like(logits)
    lib().oracle_softmax_xent_grad(_p(logits), _p(labels), _p(g), logits.shape[0],
                                   logits.shape[1])
    return g


def sgd(p, g, lr: float) -> np.ndarray:
    p = _f32(p).copy()
    g = _f32(g)
    lib().oracle_sgd(_p(p), _p(g), lr, p.size)
    return p


def mlp2_train_step(X, labels, W1, b1, W2, b2, lr: float, with_dx: bool = True) -> dict:
    """One fp32 step; returns updated params and every intermediate."""
    X = _f32(X)
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    B, I = X.shape
    Hd = W1.shape[1]
    Cc = W2.shape[1]
    out = {
        "W1": _f32(W1).copy(), "b1": _f32(b1).copy(), "W2": _f32(W2).copy(),
        "b2": _f32(b2).copy(),
        "H": np.empty((B, Hd), np.float32), "logits": np.empty((B, Cc), np.float32),
        "G2": np.empty((B, Cc), np.float32), "G1": np.empty((B, Hd), np.float32),
        "dW1": np.empty((I, Hd), np.float32), "db1": np.empty((Hd,), np.float32),
        "dW2": np.empty((Hd, Cc), np.float32), "db2": np.empty((Cc,), np.float32),
        "dX": np.empty((B, I), np.float32) if with_dx else None,
        "loss": np.zeros((1,), np.float32),
    }
    lib().oracle_mlp2_train_step(
        _p(X), _p(labels), B, I, Hd, Cc, _p(out["W1"]), _p(out["b1"]), _p(out["W2"]),
        _p(out["b2"]), lr, _p(out["H"]), _p(out["logits"]), _p(out["G2"]), _p(out["G1"]),
        _p(out["dW1"]), _p(out["db1"]), _p(out["dW2"]), _p(out["db2"]), _p(out["dX"]),
        _p(out["loss"]))
    return out


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def mlp2_loss_f64(X, labels, W1, b1, W2, b2) -> float:
    X, W1, b1, W2, b2 = map(_f64, (X, W1, b1, W2, b2))
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    return float(lib().oracle_mlp2_loss_f64(_p(X), _p(labels), X.shape[0], X.shape[1],
                                            W1.shape[1], W2.shape[1], _p(W1), _p(b1), _p(W2),
                                            _p(b2)))


def mlp2_grads_f64(X, labels, W1, b1, W2, b2) -> dict:
    X, W1, b1, W2, b2 = map(_f64, (X, W1, b1, W2, b2))
    labels = np.ascontiguousarray(labels, dtype=np.int64)
    g = {"dW1": np.empty_like(W1), "db1": np.empty_like(b1), "dW2": np.empty_like(W2),
         "db2": np.empty_like(b2), "dX": np.empty_like(X)}
    lib().oracle_mlp2_grads_f64(_p(X), _p(labels), X.shape[0], X.shape[1], W1.shape[1],
                                W2.shape[1], _p(W1), _p(b1), _p(W2), _p(b2), _p(g["dW1"]),
                                _p(g["db1"]), _p(g["dW2"]), _p(g["db2"]), _p(g["dX"]))
    return g


class IdxError(RuntimeError):
    """An IDX file the restated loader rejects; .code is the oracle's status."""

    def __init__(self, path: str, code: int):
        super().__init__(f"{path}: IDX read failed with status {code}")
        self.code = code


def idx_read_images(path: str, num: int = 0) -> np.ndarray:
    """float32 [count, rows*cols] = byte / 255 (DataLoader::load_images);
    idx_image_dims gives count, rows and cols."""
    count, rows, cols = (np.zeros(1, np.int64) for _ in range(3))
    rc = lib().oracle_idx_read_images(path.encode(), num, _p(count), _p(rows), _p(cols), None)
    if rc != 0:
        raise IdxError(path, rc)
    out = np.empty((int(count[0]), int(rows[0]) * int(cols[0])), np.float32)
    rc = lib().oracle_idx_read_images(path.encode(), num, _p(count), _p(rows), _p(cols), _p(out))
    if rc != 0:
        raise IdxError(path, rc)
    return out


def idx_image_dims(path: str, num: int = 0) -> tuple[int, int, int]:
    count, rows, cols = (np.zeros(1, np.int64) for _ in range(3))
    rc = lib().oracle_idx_read_images(path.encode(), num, _p(count), _p(rows), _p(cols), None)
    if rc != 0:
        raise IdxError(path, rc)
    return int(count[0]), int(rows[0]), int(cols[0])


def idx_read_labels(path: str, num: int = 0) -> np.ndarray:
    """int64 [count] labels as DataLoader::load_labels reads them."""
    count = np.zeros(1, np.int64)
    rc = lib().oracle_idx_read_labels(path.encode(), num, _p(count), None)
    if rc != 0:
        raise IdxError(path, rc)
    out = np.empty(int(count[0]), np.int64)
    rc = lib().oracle_idx_read_labels(path.encode(), num, _p(count), _p(out))
    if rc != 0:
        raise IdxError(path, rc)
    return out


def idx_gather(images: np.ndarray, labels: np.ndarray | None, index: np.ndarray | None,
               batch: int | None = None, divisor: float = 255.0):
    """(x float32 [batch, row_bytes], y int64 [batch]) as fdl_idx_gather."""
    images = np.ascontiguousarray(images, dtype=np.uint8)
    count, row_bytes = images.shape
    if labels is not None:
        labels = np.ascontiguousarray(labels, dtype=np.uint8)
        assert labels.shape == (count,)
    if index is not None:
        index = np.ascontiguousarray(index, dtype=np.int64)
        batch = index.size
    assert batch is not None
    x = np.empty((batch, row_bytes), np.float32)
    y = np.empty(batch, np.int64) if labels is not None else None
    lib().oracle_idx_gather(_p(images), _p(labels), count, row_bytes, _p(index), batch, divisor,
                            _p(x), _p(y))
    return x, y


def gemm_tolerance(abs_ab: np.ndarray, K: int, c0: float = 2.0) -> np.ndarray:
    """Elementwise bound c0 * (sqrt(K) + 2) * FLT_EPSILON * (|A||B| + |bias|).

    Two fp32 evaluations of the same dot product in different orders differ
    by at most a few units of sqrt(K) * eps * |A||B| in practice (the +2
    covers the bias add and the final rounding).
    """
    return c0 * (np.sqrt(max(K, 1)) + 2.0) * FLT_EPS * abs_ab + 1e-30
