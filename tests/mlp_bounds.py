"""Elementwise rounding-error bounds for one fp32 MLP training step.

For the 2-layer step (H = relu(X W1 + b1), logits = H W2 + b2, G2 =
(softmax(logits) - onehot)/B, G1 = (G2 W2^T) * [H > 0], dW1 = X^T G1,
db1 = colsum(G1), dW2 = H^T G2, db2 = colsum(G2), dX = G1 W1^T, then
p -= lr * dp), ``step_bounds`` returns, for every output, a bound on how far
ONE fp32 evaluation of the step may deviate from the exact step, whatever
its summation order.  Two evaluations (the device's and the CPU oracle's)
then differ by at most twice that.

The bound follows the errors forward through the step (first order in the
unit roundoff u = FLT_EPSILON = 2^-23, with gamma(n) = n u / (1 - n u) per
length-n dot product).  Its softmax term is what lets a p - 1 cancellation
look large against its own value: the error of p_c is proportional to p_c
itself (exp within 2 ulp, the shift by the row maximum, the row sum and the
division), so G2 = (p - 1)/B at a label whose p is near 1 carries an
absolute error of order p * u / B while being much smaller than 1/B, and
G1 = G2 W2^T and dW1 = X^T G1 inherit that absolute error, not a relative
one.  A ReLU mask that may flip (|pre-activation| within its own bound)
gets the full magnitude of the gradient it gates.

``stage_ratios`` is the same analysis between two fp32 evaluations with the
upstream differences measured instead of bounded: it checks that each
stage's difference is explained by its inputs' differences and local
rounding, which is where the p - 1 cancellation shows.

Used by tests/test_mlp_bounds_cpu.py (both bounds between the oracle and the
fp64 step or a numpy float32 step, and planted mistakes rejected) and
tests/test_mlp_bounds_gpu.py (the device step against both).
"""
from __future__ import annotations

import numpy as np

U = 2.0 ** -23  # FLT_EPSILON
FLT_MIN = 2.0 ** -126  # below this the device may flush results to zero


def gamma(n: int) -> float:
    return n * U / (1.0 - n * U)


def exact_step(X, labels, W1, b1, W2, b2, lr: float) -> dict:
    """The step in float64 from the same fp32 inputs (the reference for both sides)."""
    X, W1, b1, W2, b2 = (np.asarray(a, np.float64) for a in (X, W1, b1, W2, b2))
    B = X.shape[0]
    C = W2.shape[1]
    pre = X @ W1 + b1
    H = np.maximum(pre, 0.0)
    z = H @ W2 + b2
    m = z.max(axis=1, keepdims=True)
    e = np.exp(z - m)
    p = e / e.sum(axis=1, keepdims=True)
    valid = (labels >= 0) & (labels < C)
    onehot = np.zeros_like(p)
    onehot[np.nonzero(valid)[0], labels[valid]] = 1.0
    G2 = (p - onehot) / B
    G1 = (G2 @ W2.T) * (pre > 0)
    out = {"pre": pre, "H": H, "logits": z, "p": p, "G2": G2, "G1": G1,
           "dW1": X.T @ G1, "db1": G1.sum(axis=0), "dW2": H.T @ G2, "db2": G2.sum(axis=0),
           "dX": G1 @ W1.T}
    out["W1"] = W1 - lr * out["dW1"]
    out["b1"] = b1 - lr * out["db1"]
    out["W2"] = W2 - lr * out["dW2"]
    out["b2"] = b2 - lr * out["db2"]
    return out


def step_bounds(X, labels, W1, b1, W2, b2, lr: float, exact: dict | None = None) -> dict:
    """Bound on |fp32 step - exact step| for every output of the step."""
    ex = exact if exact is not None else exact_step(X, labels, W1, b1, W2, b2, lr)
    aX, aW1, ab1, aW2, ab2 = (np.abs(np.asarray(a, np.float64)) for a in (X, W1, b1, W2, b2))
    B, I = aX.shape
    Hd = aW1.shape[1]
    C = aW2.shape[1]
    e = {}
    # hidden pre-activation / H (relu is 1-Lipschitz)
    e["H"] = gamma(I + 2) * (aX @ aW1 + ab1)
    aH = np.abs(ex["H"]) + e["H"]
    # logits from the perturbed H
    e["logits"] = e["H"] @ aW2 + gamma(Hd + 2) * (aH @ aW2 + ab2)
    # softmax: dp_c/dz_k = p_c (delta_ck - p_k), so a logit error moves p_c by at
    # most 2 p_c max|dz|; the shift z - max rounds to within u |z - max|; exp
    # within 2 ulp; the row sum within C u; the division (or reciprocal and
    # product) within 2 u.  Relative to p_c, plus a flush-to-zero floor.
    z = ex["logits"]
    shift = np.abs(z - z.max(axis=1, keepdims=True))
    rel_p = (2.0 * e["logits"].max(axis=1, keepdims=True) + U * (shift + e["logits"]) +
             (C + 6) * U)
    e["p"] = ex["p"] * rel_p + FLT_MIN
    # G2 = (p - y) * (1/B): the subtraction and the scaling round (3 u with a
    # rounded reciprocal), on top of the carried error of p
    e["G2"] = e["p"] / B + 3.0 * U * np.abs(ex["G2"]) + FLT_MIN
    aG2 = np.abs(ex["G2"]) + e["G2"]
    # G1 = (G2 W2^T) * mask; where the mask may flip the whole product counts
    dot = e["G2"] @ aW2.T + gamma(C + 1) * (aG2 @ aW2.T)
    flip = np.abs(ex["pre"]) <= e["H"]
    e["G1"] = np.where(flip, aG2 @ aW2.T, np.where(ex["pre"] > 0, dot, 0.0)) + FLT_MIN
    aG1 = np.abs(ex["G1"]) + e["G1"]
    e["dW1"] = aX.T @ e["G1"] + gamma(B + 1) * (aX.T @ aG1) + FLT_MIN
    e["db1"] = e["G1"].sum(axis=0) + gamma(B + 1) * aG1.sum(axis=0) + FLT_MIN
    e["dW2"] = e["H"].T @ aG2 + aH.T @ e["G2"] + gamma(B + 1) * (aH.T @ aG2) + FLT_MIN
    e["db2"] = e["G2"].sum(axis=0) + gamma(B + 1) * aG2.sum(axis=0) + FLT_MIN
    e["dX"] = e["G1"] @ aW1.T + gamma(Hd + 1) * (aG1 @ aW1.T) + FLT_MIN
    # p - lr * g: the carried gradient error, the product and the subtraction
    for name, grad in (("W1", "dW1"), ("b1", "db1"), ("W2", "dW2"), ("b2", "db2")):
        e[name] = (lr * e[grad] * (1 + U) + U * lr * (np.abs(ex[grad]) + e[grad]) +
                   U * (np.abs(ex[name]) + lr * e[grad]) + FLT_MIN)
    return e


OUTPUTS = ["H", "logits", "G2", "G1", "dW1", "db1", "dW2", "db2", "dX", "W1", "b1", "W2", "b2"]


def numpy_step_f32(X, labels, W1, b1, W2, b2, lr: float) -> dict:
    """A second fp32 evaluation of the step: numpy's float32 products (its own
    summation order) and numpy's float32 exp (its own implementation, not the
    C library's expf), as the device differs from the oracle."""
    f = np.float32
    B = X.shape[0]
    C = W2.shape[1]
    H = np.maximum(X @ W1 + b1, f(0))
    z = H @ W2 + b2
    e = np.exp(z - z.max(axis=1, keepdims=True))
    p = e * (f(1) / e.sum(axis=1, keepdims=True, dtype=f))
    valid = (labels >= 0) & (labels < C)
    rows = np.nonzero(valid)[0]
    G2 = p.copy()
    G2[rows, labels[rows]] -= f(1)
    G2 = G2 * (f(1) / f(B))
    G1 = np.where(H > 0, G2 @ W2.T, f(0))
    out = {"H": H, "logits": z, "G2": G2, "G1": G1, "dW1": X.T @ G1, "db1": G1.sum(axis=0),
           "dW2": H.T @ G2, "db2": G2.sum(axis=0), "dX": G1 @ W1.T}
    for name, grad, val in (("W1", "dW1", W1), ("b1", "db1", b1), ("W2", "dW2", W2),
                            ("b2", "db2", b2)):
        out[name] = val - f(lr) * out[grad]
    return out


def stage_ratios(a: dict, b: dict, X, labels, W1, b1, W2, b2, lr: float) -> dict:
    """Two fp32 evaluations a and b of one step, compared stage by stage.

    Each stage's difference must be explained by the MEASURED difference of
    its inputs carried through the stage, plus both sides' local rounding:
      logits: |dH| |W2| + 2 gamma(H+2) (|H||W2| + |b2|)
      G2:     (2 p max_row|dlogits| + 2 p u (|z - max| + C + 6)) / B + 6 u |G2|
              (the softmax error is proportional to p: at a label whose p is
              near 1, G2 = (p - 1)/B is small but its error is not)
      G1:     |dG2| |W2|^T + 2 gamma(C+1) |G2||W2|^T, or the full magnitude
              where the two ReLU masks disagree
      dW1:    |X|^T |dG1| + 2 gamma(B+1) |X|^T|G1|   (db1, dW2, db2, dX alike)
      params: lr |dgrad| + u (lr (|g_a| + |g_b|) + |p_a| + |p_b|)
    Returns max |a - b| / bound per stage (<= 1 means explained)."""
    d = lambda k: np.abs(np.asarray(a[k], np.float64) - np.asarray(b[k], np.float64))  # noqa: E731
    mx = lambda k: np.maximum(np.abs(np.asarray(a[k], np.float64)),  # noqa: E731
                              np.abs(np.asarray(b[k], np.float64)))
    aX, aW1, ab1, aW2, ab2 = (np.abs(np.asarray(v, np.float64)) for v in (X, W1, b1, W2, b2))
    B, I = aX.shape
    Hd = aW1.shape[1]
    C = aW2.shape[1]
    bound = {}
    bound["H"] = 2 * gamma(I + 2) * (aX @ aW1 + ab1) + FLT_MIN
    aH = mx("H")
    bound["logits"] = d("H") @ aW2 + 2 * gamma(Hd + 2) * (aH @ aW2 + ab2) + FLT_MIN
    z = np.asarray(a["logits"], np.float64)
    ez = np.exp(z - z.max(axis=1, keepdims=True))
    p = ez / ez.sum(axis=1, keepdims=True)
    dz = d("logits").max(axis=1, keepdims=True)
    shift = np.abs(z - z.max(axis=1, keepdims=True))
    bound["G2"] = ((2 * p * dz + 2 * p * U * (shift + C + 6)) / B + 6 * U * mx("G2") +
                   2 * FLT_MIN)
    aG2, dG2 = mx("G2"), d("G2")
    masks_differ = (np.asarray(a["H"]) > 0) != (np.asarray(b["H"]) > 0)
    carried = dG2 @ aW2.T + 2 * gamma(C + 1) * (aG2 @ aW2.T)
    bound["G1"] = np.where(masks_differ, aG2 @ aW2.T + dG2 @ aW2.T, carried) + 2 * FLT_MIN
    aG1, dG1 = mx("G1"), d("G1")
    bound["dW1"] = aX.T @ dG1 + 2 * gamma(B + 1) * (aX.T @ aG1) + 2 * FLT_MIN
    bound["db1"] = dG1.sum(axis=0) + 2 * gamma(B + 1) * aG1.sum(axis=0) + 2 * FLT_MIN
    bound["dW2"] = (d("H").T @ aG2 + aH.T @ dG2 + 2 * gamma(B + 1) * (aH.T @ aG2) +
                    2 * FLT_MIN)
    bound["db2"] = dG2.sum(axis=0) + 2 * gamma(B + 1) * aG2.sum(axis=0) + 2 * FLT_MIN
    if a.get("dX") is not None and b.get("dX") is not None:
        bound["dX"] = dG1 @ aW1.T + 2 * gamma(Hd + 1) * (aG1 @ aW1.T) + 2 * FLT_MIN
    for name, grad in (("W1", "dW1"), ("b1", "db1"), ("W2", "dW2"), ("b2", "db2")):
        bound[name] = (lr * d(grad) * (1 + U) + U * (lr * 2 * mx(grad) + 2 * mx(name)) +
                       2 * FLT_MIN)
    return {k: float(np.max(d(k) / v)) if v.size else 0.0 for k, v in bound.items()}


def worst_ratio(got: dict, ex: dict, bounds: dict, names=OUTPUTS) -> dict:
    """max |got - exact| / bound per output (<= 1 means within the bound)."""
    out = {}
    for n in names:
        if got.get(n) is None:
            continue
        d = np.abs(np.asarray(got[n], np.float64) - ex[n])
        out[n] = float(np.max(d / bounds[n])) if d.size else 0.0
    return out
