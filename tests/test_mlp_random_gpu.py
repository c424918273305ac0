"""Seeded random sweep of fdl_mlp2_train_step against the oracle step.

Shapes are drawn across the head kernel's dispatch boundaries (classes up to
40 against the 16- and 32-class paddings, hidden up to 1100 against the 512
and 1024 limits, batches that are not multiples of its 8 rows, dW1 too small
for its records, hidden values that do and do not fit the fused head and dX
kernel) so the three-, four- and six-launch steps are all reached, with and
without dX, and some labels outside [0, classes) (left out of the
loss, as the reference's cross_entropy does).  Bar: every intermediate and
updated parameter within 1e-4 of the fp32 oracle step, normwise (the path's
"max relative error <= 1e-4" criterion), with the products and column sums
measured against the magnitudes of their terms; loss within 1e-5.  The
structured shape tests hold the same outputs to 2e-5; over thousands of
random shapes a G2 entry p - 1 with p near 1, which the device's and the
host's expf round apart, carries differences of a few 1e-5 through G1 into
dW1, which is why the sweep uses the criterion itself.
"""
import numpy as np
import pytest

import oracle
from tests.gpu_helpers import say
from tests.test_mlp_gpu import _step_gpu

pytestmark = pytest.mark.gpu

N_CASES = 120


def _draw(g):
    B = int(g.choice([1, 2, 7, 8, 9, 31, 64, 100, 255, 256, 300]))
    I = int(np.exp(g.uniform(0, np.log(800))))
    H = int(g.choice([1, 3, 16, 100, 255, 256, 257, 511, 512, 513, 700, 1024, 1025, 1100]))
    C = int(g.choice([1, 2, 9, 10, 15, 16, 17, 31, 32, 33, 40]))
    with_dx = bool(g.integers(0, 4) > 0)
    invalid = bool(g.integers(0, 4) == 0)
    return B, I, H, C, with_dx, invalid


def case_inputs(case):
    """Inputs of sweep case `case` (seeded by the case number):
    (X, labels, W1, b1, W2, b2, with_dx, invalid)."""
    g = np.random.default_rng(2000 + case)
    B, I, H, C, with_dx, invalid = _draw(g)
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    if invalid:
        labels[::5] = -1
        labels[2::7] = C
    W1 = g.uniform(-np.sqrt(6 / I), np.sqrt(6 / I), (I, H)).astype(np.float32)
    W2 = g.uniform(-np.sqrt(6 / H), np.sqrt(6 / H), (H, C)).astype(np.float32)
    b1 = (g.standard_normal(H) * 0.1).astype(np.float32)
    b2 = (g.standard_normal(C) * 0.1).astype(np.float32)
    return X, labels, W1, b1, W2, b2, with_dx, invalid


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_mlp_step(device, case):
    X, labels, W1, b1, W2, b2, with_dx, invalid = case_inputs(case)
    (B, I), H, C = X.shape, W1.shape[1], W2.shape[1]
    say(f"random mlp2 step case {case}: B={B} I={I} H={H} C={C} dx={with_dx} invalid={invalid}")
    gpu = _step_gpu(X, labels, W1, b1, W2, b2, 0.05, with_dx=with_dx)
    ref = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, 0.05, with_dx=with_dx)
    names = ["H", "logits", "G2", "G1", "dW1", "db1", "dW2", "db2", "W1", "b1", "W2", "b2"]
    if with_dx:
        names.append("dX")
    # Products and column sums are measured against the magnitudes of their
    # terms (|A||B| + |bias|, sum of |terms|), the scale on which two
    # evaluation orders differ: their terms can cancel (a row of G2 sums to 0
    # for a valid label), and a G2 entry p - 1 with p near 1 carries the
    # device's and the host's expf apart by more than its own size suggests.
    r = {k: np.abs(v.astype(np.float64)) for k, v in ref.items() if v is not None}
    aX, aW1, aW2 = (np.abs(v.astype(np.float64)) for v in (X, W1, W2))
    mag = {"H": aX @ aW1 + np.abs(b1), "logits": r["H"] @ aW2 + np.abs(b2),
           "G1": r["G2"] @ aW2.T, "dW1": aX.T @ r["G1"], "dW2": r["H"].T @ r["G2"],
           "dX": r["G1"] @ aW1.T, "db1": r["G1"].sum(axis=0), "db2": r["G2"].sum(axis=0)}
    for name in names:
        a = gpu[name].astype(np.float64)
        b = ref[name].astype(np.float64)
        assert np.all(np.isfinite(a)), name
        scale = np.max(mag[name]) if name in mag else np.max(np.abs(b))
        err = np.max(np.abs(a - b)) / max(1e-30, scale)
        assert err <= 1e-4, f"{name}: normwise error {err:.2e}"
    assert abs(gpu["loss"][0] - ref["loss"][0]) <= 1e-5
