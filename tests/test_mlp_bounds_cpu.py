"""The MLP step's derived error bound (tests/mlp_bounds.py), pinned on the CPU.

* The fp64 restatement of the step agrees with the oracle's fp64 gradients
  (oracle_mlp2_grads_f64, itself pinned by finite differences).
* The fp32 oracle step stays within the bound of the exact step, on the two
  shapes where a 2000-shape GPU sweep found the largest normwise differences
  (sweep cases 309: B=31 I=105 H=700 C=2, db2; 1453: B=9 I=608 H=1 C=31, G1
  and dW1), on the committed sweep's shapes and on BASELINE config 2.
* The stage chain (each stage's difference explained by its inputs'
  measured differences and local rounding) holds between the oracle and a
  numpy float32 step, whose exp is not the C library's expf: the CPU
  instance of the device-vs-oracle comparison.
* Neither is vacuous: planted mistakes (the label's -1 on the wrong class, a
  dropped ReLU mask, a dropped batch row in dW1) exceed the worst-case
  bound; an exp 1e-4 off exceeds the chain's G2 stage and a learning rate
  1% off its W1 stage.
"""
import numpy as np
import pytest

import oracle
from tests.mlp_bounds import (exact_step, numpy_step_f32, stage_ratios, step_bounds,
                               worst_ratio)
from tests.test_mlp_random_gpu import N_CASES, case_inputs

LR = 0.05
FUZZ_CASES = [309, 1453]


def _c2():
    g = np.random.default_rng(2)
    B, I, H, C = 256, 784, 256, 10
    X = g.random((B, I), dtype=np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-(6 / I) ** 0.5, (6 / I) ** 0.5, (I, H)).astype(np.float32)
    W2 = g.uniform(-(6 / H) ** 0.5, (6 / H) ** 0.5, (H, C)).astype(np.float32)
    return X, labels, W1, np.zeros(H, np.float32), W2, np.zeros(C, np.float32), True, False


def _inputs(case):
    return _c2() if case == "c2" else case_inputs(case)


@pytest.mark.parametrize("case", FUZZ_CASES + ["c2", 0, 7, 33, 64, 101])
def test_exact_step_matches_oracle_f64(case):
    X, labels, W1, b1, W2, b2, _, _ = _inputs(case)
    ex = exact_step(X, labels, W1, b1, W2, b2, LR)
    g = oracle.mlp2_grads_f64(X, labels, W1, b1, W2, b2)
    for k in ("dW1", "db1", "dW2", "db2", "dX"):
        scale = max(1e-300, float(np.max(np.abs(g[k]))))
        assert np.max(np.abs(ex[k] - g[k])) <= 1e-12 * scale, k


@pytest.mark.parametrize("case", FUZZ_CASES + ["c2"] + list(range(N_CASES)))
def test_oracle_step_within_bound(case):
    X, labels, W1, b1, W2, b2, with_dx, _ = _inputs(case)
    ref = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, LR, with_dx=with_dx)
    ex = exact_step(X, labels, W1, b1, W2, b2, LR)
    bd = step_bounds(X, labels, W1, b1, W2, b2, LR, ex)
    r = worst_ratio(ref, ex, bd)
    assert max(r.values()) <= 1.0, r


@pytest.mark.parametrize("case", FUZZ_CASES + ["c2"] + list(range(N_CASES)))
def test_stage_chain_numpy_vs_oracle(case):
    # numpy's float32 exp and products against the oracle's expf and loops: a
    # CPU instance of two fp32 evaluations that round apart
    X, labels, W1, b1, W2, b2, _, _ = _inputs(case)
    ref = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, LR, with_dx=True)
    npy = numpy_step_f32(X, labels, W1, b1, W2, b2, LR)
    r = stage_ratios(npy, ref, X, labels, W1, b1, W2, b2, LR)
    assert max(r.values()) <= 1.0, r


@pytest.mark.parametrize("case", FUZZ_CASES + ["c2"])
def test_bounds_reject_planted_mistakes(case):
    X, labels, W1, b1, W2, b2, _, _ = _inputs(case)
    ref = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, LR, with_dx=True)
    ex = exact_step(X, labels, W1, b1, W2, b2, LR)
    bd = step_bounds(X, labels, W1, b1, W2, b2, LR, ex)
    B, C = ref["G2"].shape
    X64, W1_64, W2_64 = (a.astype(np.float64) for a in (X, W1, W2))
    rows = np.nonzero((labels >= 0) & (labels < C))[0]

    def rejected(name, value):
        return worst_ratio({name: value}, ex, bd, [name])[name] > 1.0

    # The worst-case bound against the exact step:
    # the label's -1 on the neighbouring class
    if C > 1 and rows.size:
        moved = ex["G2"].copy()
        moved[rows, labels[rows]] += 1.0 / B
        moved[rows, (labels[rows] + 1) % C] -= 1.0 / B
        assert rejected("G2", moved)
    # the ReLU mask dropped in G1 (where it gates something)
    nomask = ex["G2"] @ W2_64.T
    if np.any((ex["pre"] <= 0) & (np.abs(nomask) > 0)):
        assert rejected("G1", nomask)
    # one batch row missing from dW1
    if B > 1 and np.any(ex["G1"][-1] != 0):
        assert rejected("dW1", X64[:-1].T @ ex["G1"][:-1])

    # The stage chain between two fp32 evaluations: a learning rate 1% off in
    # the second evaluation's W1 update ...
    f = np.float32
    bad = numpy_step_f32(X, labels, W1, b1, W2, b2, LR)
    if np.any(bad["dW1"] != 0):
        bad["W1"] = W1 - f(1.01 * LR) * bad["dW1"]
        assert stage_ratios(bad, ref, X, labels, W1, b1, W2, b2, LR)["W1"] > 1.0
    # ... and an exp 1e-4 off (relative), G2 recomputed from it
    bad = numpy_step_f32(X, labels, W1, b1, W2, b2, LR)
    z = bad["logits"]
    e = np.exp(z - z.max(axis=1, keepdims=True)) * f(1 + 1e-4)
    p = e * (f(1) / e.sum(axis=1, keepdims=True, dtype=f)) * f(1 + 1e-4)
    g2 = p.copy()
    g2[rows, labels[rows]] -= f(1)
    bad["G2"] = g2 * (f(1) / f(B))
    r = stage_ratios(bad, ref, X, labels, W1, b1, W2, b2, LR)
    assert r["G2"] > 1.0, r
