"""Writes the golden fixtures in tests/golden/ from the CPU oracle.

Inputs are regenerated from numpy PCG64 seeds in the tests; the fixtures hold
the oracle's outputs (for config 1 with SHA-256 digests of the inputs, as a
guard that the generator still yields the same arrays).  Run from the repo root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def config1():
    # M=256, K=784, N=128; A ~ U[0,1), B ~ N(0, sqrt(2/784)); seed 1
    g = np.random.default_rng(1)
    M, K, N = 256, 784, 128
    A = g.random((1, M, K)).astype(np.float32)
    B = (g.standard_normal((1, K, N)) * np.sqrt(2.0 / 784)).astype(np.float32)
    C32 = oracle.sgemm_ex(0, 0, A, B, M, N, K)[0]
    C64, S64 = oracle.sgemm_ex_f64(0, 0, A, B, M, N, K)
    assert np.array_equal(C32, oracle.gemm_cpu(A[0], B[0]))
    import hashlib

    np.savez_compressed(os.path.join(HERE, "config1_gemm.npz"), C32=C32, C64=C64[0],
                        sha_A=np.frombuffer(hashlib.sha256(A.tobytes()).digest(), np.uint8),
                        sha_B=np.frombuffer(hashlib.sha256(B.tobytes()).digest(), np.uint8))


def mlp_small():
    # A reduced 64-32-10 MLP at batch 16, one SGD step with lr 0.1; seed 2
    g = np.random.default_rng(2)
    B, I, H, C = 16, 64, 32, 10
    X = g.random((B, I)).astype(np.float32)
    labels = g.integers(0, C, B).astype(np.int64)
    W1 = g.uniform(-np.sqrt(6 / I), np.sqrt(6 / I), (I, H)).astype(np.float32)
    b1 = np.zeros(H, np.float32)
    W2 = g.uniform(-np.sqrt(6 / H), np.sqrt(6 / H), (H, C)).astype(np.float32)
    b2 = np.zeros(C, np.float32)
    out = oracle.mlp2_train_step(X, labels, W1, b1, W2, b2, 0.1)
    np.savez_compressed(os.path.join(HERE, "mlp2_small_step.npz"), X=X, labels=labels, W1=W1,
                        b1=b1, W2=W2, b2=b2, lr=np.float32(0.1),
                        **{f"out_{k}": v for k, v in out.items() if v is not None})


if __name__ == "__main__":
    config1()
    mlp_small()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
