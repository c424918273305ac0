"""GPU parity of the MLP-step kernels and of fdl_mlp2_train_step.

Elementwise kernels (ReLU, ReLU backward, row bias, SGD) are bit-exact with
the oracle; reductions (colsum, softmax, cross-entropy) are within 1e-6
relative of it (different summation order); the full step matches the fp32
oracle step within the GEMM bound propagated through one update.
"""
import os

import numpy as np
import pytest

import fast_dl_amd.capi as capi
import oracle
from tests.conftest import rng
from tests.gpu_helpers import dev, host, say, stream

pytestmark = pytest.mark.gpu


def test_relu_fixture_and_backward(device):
    import torch

    # tests/nn/relu_module_test.cpp:22-29
    x = np.array([-2.0, -0.5, 0.0, 1.5, 3.0, -4.0], np.float32)
    dx = dev(x)
    dy = torch.empty_like(dx)
    say("relu fixture")
    capi.relu(dx.data_ptr(), dy.data_ptr(), x.size, stream())
    assert np.array_equal(host(dy), [0.0, 0.0, 0.0, 1.5, 3.0, 0.0])
    g = rng(1)
    a = g.standard_normal(100003).astype(np.float32)
    gr = g.standard_normal(100003).astype(np.float32)
    da, dg = dev(a), dev(gr)
    out = torch.empty_like(da)
    say("relu large + backward")
    capi.relu(da.data_ptr(), out.data_ptr(), a.size, stream())
    assert np.array_equal(host(out), oracle.relu(a))
    capi.relu_backward(dg.data_ptr(), da.data_ptr(), out.data_ptr(), a.size, stream())
    assert np.array_equal(host(out), oracle.relu_backward(gr, a))


def test_add_row_bias_and_sgd(device):
    g = rng(2)
    rows, cols = 129, 77
    y = g.standard_normal((rows, cols)).astype(np.float32)
    b = g.standard_normal(cols).astype(np.float32)
    dy, db = dev(y), dev(b)
    say("add_row_bias")
    capi.add_row_bias(dy.data_ptr(), db.data_ptr(), rows, cols, stream())
    assert np.array_equal(host(dy), y + b)
    p = g.standard_normal(5000).astype(np.float32)
    d = g.standard_normal(5000).astype(np.float32)
    dp, dd = dev(p), dev(d)
    say("sgd_update")
    capi.sgd_update(dp.data_ptr(), dd.data_ptr(), 0.01, p.size, stream())
    assert np.array_equal(host(dp), oracle.sgd(p, d, 0.01))


@pytest.mark.parametrize("rows,cols", [(1, 1), (256, 10), (37, 300), (5, 4097)])
def test_colsum(device, rows, cols):
    import torch

    g = rng(rows + cols)
    x = g.standard_normal((rows, cols)).astype(np.float32)
    dx = dev(x)
    out = torch.full((cols,), float("nan"), device="cuda")
    say(f"colsum {rows}x{cols}")
    capi.colsum(dx.data_ptr(), out.data_ptr(), rows, cols, stream())
    ref = oracle.colsum(x)
    bound = 2 * (rows + 2) * oracle.FLT_EPS * np.abs(x).astype(np.float64).sum(0) + 1e-30
    assert np.all(np.abs(host(out) - ref) <= bound)


def test_softmax_fixture_and_random(device):
    import torch

    # tests/tensor/softmax_tensor_test.cpp:43-46 with its 1e-4 rule and unit row sums
    x = np.array([[1, 2, 3, 4], [1, 3, 2, 0]], np.float32)
    for arr in (x, rng(3).standard_normal((333, 1000)).astype(np.float32) * 5):
        d = dev(arr)
        out = torch.empty_like(d)
        say(f"softmax {arr.shape}")
        capi.softmax(d.data_ptr(), out.data_ptr(), arr.shape[0], arr.shape[1], stream())
        y = host(out)
        ref = oracle.softmax(arr)
        assert np.max(np.abs(y - ref)) < 1e-4  # the reference test's own rule
        # elementwise: exp differs by a few ulp between libraries and the row sum
        # by ~sqrt(cols) roundings
        bound = (8.0 + 2.0 * np.sqrt(arr.shape[1])) * oracle.FLT_EPS * ref + 1e-30
        assert np.all(np.abs(y - ref) <= bound)
        assert np.all(np.abs(y.sum(1) - 1.0) < 1e-4)


def test_cross_entropy_fixture(device):
    import torch

    # tests/tensor/cross_entropy_tensor_test.cpp:40-44 -> 0.4076059 (abs 1e-4)
    z = np.array([[1, 2, 3], [1, 3, 2]], np.float32)
    lab = np.array([2, 1], np.int64)
    dz, dl = dev(z), dev(lab)
    loss = torch.full((1,), float("nan"), device="cuda")
    grad = torch.empty_like(dz)
    say("softmax_xent fixture")
    capi.softmax_xent(dz.data_ptr(), dl.data_ptr(), loss.data_ptr(), grad.data_ptr(), 2, 3,
                      stream())
    assert abs(host(loss)[0] - 0.4076059) < 1e-4
    assert np.max(np.abs(host(grad) - oracle.softmax_xent_grad(z, lab))) < 1e-7


@pytest.mark.parametrize("batch,classes", [(256, 10), (1000, 37), (3, 1)])
def test_softmax_xent_random(device, batch, classes):
    import torch

    g = rng(batch * classes)
    z = (g.standard_normal((batch, classes)) * 3).astype(np.float32)
    lab = g.integers(0, classes, batch).astype(np.int64)
    lab[::17] = -1  # invalid labels: skipped in the loss, still counted in the batch
    dz, dl = dev(z), dev(lab)
    loss = torch.full((1,), float("nan"), device="cuda")
    grad = torch.empty_like(dz)
    say(f"softmax_xent {batch}x{classes}")
    capi.softmax_xent(dz.data_ptr(), dl.data_ptr(), loss.data_ptr(), grad.data_ptr(), batch,
                      classes, stream())
    ref = oracle.cross_entropy(z, lab)
    assert abs(host(loss)[0] - ref) <= 1e-5 * max(1.0, abs(ref))
    assert np.max(np.abs(host(grad) - oracle.softmax_xent_grad(z, lab))) < 1e-7


def _step_gpu(X, labels, W1, b1, W2, b2, lr, with_dx=True):
    import torch

    B, I = X.shape
    Hd, Cc = W1.shape[1], W2.shape[1]
    t = {k: dev(v.copy()) for k, v in dict(X=X, labels=labels, W1=W1, b1=b1, W2=W2, b2=b2).items()}
    for name, shape in dict(H=(B, Hd), logits=(B, Cc), G2=(B, Cc), G1=(B, Hd), dW1=(I, Hd),
                            db1=(Hd,), dW2=(Hd, Cc), db2=(Cc,), dX=(B, I), loss=(1,)).items():
        t[name] = torch.full(shape, float("nan"), device="cuda")
    ptr = {k: v.data_ptr() for k, v in t.items()}
    capi.mlp2_train_step(ptr["X"], ptr["labels"], B, I, Hd, Cc, ptr["W1"], ptr["b1"], ptr["W2"],
                         ptr["b2"], lr, ptr["H"], ptr["logits"], ptr["G2"], ptr["G1"],
                         ptr["dW1"], ptr["db1"], ptr["dW2"], ptr["db2"],
                         ptr["dX"] if with_dx else None, ptr["loss"], stream())
    torch.cuda.synchronize()
    return {k: host(v) for k, v in t.items()}


def _compare_step(gpu, ref, scale_tol=2e-5):
    for name in ("H", "logits", "G2", "G1", "dW1", "db1", "dW2", "db2", "dX", "W1", "b1", "W2",
                 "b2"):
        a = gpu[name].astype(np.float64)
        b = ref[name].astype(np.float64)
        assert np.all(np.isfinite(a)), name
        err = np.max(np.abs(a - b)) / max(1e-30, np.max(np.abs(b)))
        assert err <= scale_tol, f"{name}: normwise error {err:.2e}"
    assert abs(gpu["loss"][0] - ref["loss"][0]) <= 1e-5


def test_mlp_small_golden(device):
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "mlp2_small_step.npz"))
    args = [gold[k] for k in ("X", "labels", "W1", "b1", "W2", "b2")]
    say("mlp2 small golden step")
    gpu = _step_gpu(*args, float(gold["lr"]))
    ref = {k[4:]: gold[k] for k in gold.files if k.startswith("out_")}
    _compare_step(gpu, ref)


def test_mlp_config2_step(device):
    # 784-256-10 at batch 256, X ~ U[0,1), labels U{0..9},
    # He (Kaiming-uniform, +-sqrt(6/fan_in)) weights as nn::Linear's default, zero bias, lr 0.1
    g = rng(2)
    B, I, H, C = 256, 784, 256, 10
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-np.sqrt(6 / I), np.sqrt(6 / I), (I, H)).astype(np.float32)
    W2 = g.uniform(-np.sqrt(6 / H), np.sqrt(6 / H), (H, C)).astype(np.float32)
    b1 = np.zeros(H, np.float32)
    b2 = np.zeros(C, np.float32)
    say("mlp2 config2 step")
    gpu = _step_gpu(X, labels, W1, b1, W2, b2, 0.1)
    ref = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, 0.1)
    _compare_step(gpu, ref)
    # ten more steps stay in agreement (loss decreases on a fixed batch)
    ref_state = {k: ref[k] for k in ("W1", "b1", "W2", "b2")}
    gpu_state = {k: gpu[k] for k in ("W1", "b1", "W2", "b2")}
    losses = []
    for _ in range(10):
        gpu = _step_gpu(X, labels, gpu_state["W1"], gpu_state["b1"], gpu_state["W2"],
                        gpu_state["b2"], 0.1, with_dx=False)
        ref = oracle.mlp2_train_step(X, labels, ref_state["W1"], ref_state["b1"],
                                     ref_state["W2"], ref_state["b2"], 0.1, with_dx=False)
        gpu_state = {k: gpu[k] for k in ("W1", "b1", "W2", "b2")}
        ref_state = {k: ref[k] for k in ("W1", "b1", "W2", "b2")}
        losses.append(float(gpu["loss"][0]))
        assert abs(gpu["loss"][0] - ref["loss"][0]) <= 1e-4
    for k in ("W1", "b1", "W2", "b2"):
        err = np.max(np.abs(gpu_state[k] - ref_state[k])) / np.max(np.abs(ref_state[k]))
        assert err <= 1e-4, k
    assert losses[-1] < losses[0]


@pytest.mark.parametrize("B,I,H,C", [(300, 50, 20, 10), (1, 8, 4, 3), (17, 9, 256, 16),
                                     (24, 6, 1000, 12), (260, 12, 300, 20), (64, 30, 17, 40),
                                     (16, 8, 1100, 5), (10, 5, 600, 20), (64, 1, 2, 10)])
def test_mlp_step_shapes(device, B, I, H, C):
    # Four-launch step (head kernel): a batch that is not a multiple of the
    # head's 8 rows per block, batch 1, up to 16 classes with hidden up to 256
    # and up to 1024, up to 32 classes with hidden up to 512.  Six-launch
    # step: a class count past 32 (separate loss and bias-gradient kernels),
    # hidden past 1024, 17-32 classes with hidden past 512, and a dW1 too
    # small to hold the head's per-block records.
    g = rng(B * 7 + C)
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-np.sqrt(6 / I), np.sqrt(6 / I), (I, H)).astype(np.float32)
    W2 = g.uniform(-np.sqrt(6 / H), np.sqrt(6 / H), (H, C)).astype(np.float32)
    b1 = (g.standard_normal(H) * 0.1).astype(np.float32)
    b2 = (g.standard_normal(C) * 0.1).astype(np.float32)
    say(f"mlp2 step B={B} I={I} H={H} C={C}")
    gpu = _step_gpu(X, labels, W1, b1, W2, b2, 0.05)
    ref = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, 0.05)
    _compare_step(gpu, ref)


def _alloc_step(X, labels, W1, b1, W2, b2):
    import torch

    B, I = X.shape
    Hd, Cc = W1.shape[1], W2.shape[1]
    t = {k: dev(v.copy()) for k, v in dict(X=X, labels=labels, W1=W1, b1=b1, W2=W2, b2=b2).items()}
    for name, shape in dict(H=(B, Hd), logits=(B, Cc), G2=(B, Cc), G1=(B, Hd), dW1=(I, Hd),
                            db1=(Hd,), dW2=(Hd, Cc), db2=(Cc,), dX=(B, I), loss=(1,)).items():
        t[name] = torch.full(shape, float("nan"), device="cuda")
    p = {k: v.data_ptr() for k, v in t.items()}
    args = (p["X"], p["labels"], B, I, Hd, Cc, p["W1"], p["b1"], p["W2"], p["b2"], 0.1, p["H"],
            p["logits"], p["G2"], p["G1"], p["dW1"], p["db1"], p["dW2"], p["db2"], p["dX"],
            p["loss"])
    return t, args


def test_mlp_graph_replays_match_eager(device):
    # Every replay of the captured step must equal the eager step exactly (all
    # kernels are deterministic), with eager work and synchronisations between
    # the replays.
    import torch

    g = rng(77)
    B, I, H, C = 256, 784, 256, 10
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-np.sqrt(6 / I), np.sqrt(6 / I), (I, H)).astype(np.float32)
    W2 = g.uniform(-np.sqrt(6 / H), np.sqrt(6 / H), (H, C)).astype(np.float32)
    b1 = np.zeros(H, np.float32)
    b2 = np.zeros(C, np.float32)
    te, eargs = _alloc_step(X, labels, W1, b1, W2, b2)
    tg, gargs = _alloc_step(X, labels, W1, b1, W2, b2)
    s = stream()
    say("mlp2 graph create")
    handle = capi.mlp2_graph_create(*gargs, s)
    try:
        for step in range(5):
            say(f"mlp2 graph replay {step}")
            capi.mlp2_train_step(*eargs, s)
            capi.mlp2_graph_launch(handle, s)
            torch.cuda.synchronize()
            junk = torch.randn(1000, device="cuda").sum().item()  # unrelated eager work
            assert np.isfinite(junk)
            for k in ("W1", "b1", "W2", "b2", "loss", "dX", "G1", "dW1", "db1"):
                assert torch.equal(te[k], tg[k]), f"replay {step}: {k} differs"
    finally:
        capi.mlp2_graph_destroy(handle)


def test_mlp_multi_step_graph_matches_eager_steps(device):
    # A graph of three consecutive steps, replayed twice, leaves every buffer
    # as six eager steps do (each step reads what the previous one updated).
    import torch

    g = rng(78)
    B, I, H, C = 256, 784, 256, 10
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-np.sqrt(6 / I), np.sqrt(6 / I), (I, H)).astype(np.float32)
    W2 = g.uniform(-np.sqrt(6 / H), np.sqrt(6 / H), (H, C)).astype(np.float32)
    b1 = np.zeros(H, np.float32)
    b2 = np.zeros(C, np.float32)
    te, eargs = _alloc_step(X, labels, W1, b1, W2, b2)
    tg, gargs = _alloc_step(X, labels, W1, b1, W2, b2)
    s = stream()
    say("mlp2 graph create (3 steps)")
    handle = capi.mlp2_graph_create_steps(3, *gargs, s)
    try:
        for rep in range(2):
            say(f"mlp2 3-step graph replay {rep}")
            for _ in range(3):
                capi.mlp2_train_step(*eargs, s)
            capi.mlp2_graph_launch(handle, s)
            torch.cuda.synchronize()
            junk = torch.randn(1000, device="cuda").sum().item()  # unrelated eager work
            assert np.isfinite(junk)
            for k in ("W1", "b1", "W2", "b2", "loss", "dX", "G1", "dW1", "db1", "dW2", "db2"):
                assert torch.equal(te[k], tg[k]), f"replay {rep}: {k} differs"
    finally:
        capi.mlp2_graph_destroy(handle)


def test_random_fills(device):
    import torch

    n = 1 << 20
    a = torch.empty(n, device="cuda")
    b = torch.empty(n, device="cuda")
    say("fill_uniform / fill_normal")
    capi.fill_uniform(a.data_ptr(), n, -2.0, 3.0, 1234, stream())
    capi.fill_uniform(b.data_ptr(), n, -2.0, 3.0, 1234, stream())
    ua, ub = host(a), host(b)
    assert np.array_equal(ua, ub)  # same seed, same values (tensor_uniform_test semantics)
    assert ua.min() > -2.0 and ua.max() <= 3.0
    assert abs(ua.mean() - 0.5) < 0.01
    capi.fill_uniform(b.data_ptr(), n, -2.0, 3.0, 1235, stream())
    assert not np.array_equal(ua, host(b))
    capi.fill_normal(a.data_ptr(), n, 1.0, 2.0, 7, stream())
    z = host(a)
    assert abs(z.mean() - 1.0) < 0.01 and abs(z.std() - 2.0) < 0.01
    assert np.all(np.isfinite(z))
