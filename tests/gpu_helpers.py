"""Helpers for the GPU parity tests: device buffers via torch, calls via the C-ABI."""
from __future__ import annotations

import sys

import numpy as np

import fast_dl_amd.capi as capi
import oracle


def say(msg: str) -> None:
    """Name the case before a GPU step, so a crash still identifies it."""
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def stream() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream


def operands(g: np.random.Generator, ta, tb, M, N, K, batch, dist="normal", scale=1.0):
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    if dist == "normal":
        A = (g.standard_normal(a_shape) * scale).astype(np.float32)
        B = (g.standard_normal(b_shape) * scale).astype(np.float32)
    elif dist == "int":
        A = g.integers(-4, 5, a_shape).astype(np.float32)
        B = g.integers(-4, 5, b_shape).astype(np.float32)
    else:
        raise ValueError(dist)
    return A, B


def gpu_sgemm(ta, tb, A, B, M, N, K, batch=1, bias=None, aux=None, epilogue=0,
              kernel=capi.KERNEL_AUTO, lda=None, ldb=None, ldc=None, workspace=None):
    """Run fdl_sgemm_ex_select on packed operands; returns C [batch, M, N] on the host.

    C is pre-filled with NaN so an element the kernel fails to write is caught.
    With ``workspace`` (a byte count) the call is fdl_sgemm_ex_ws with a
    NaN-filled workspace of that size instead.
    """
    import torch

    a_cols = M if ta else K
    b_cols = K if tb else N
    lda = lda or max(1, a_cols)
    ldb = ldb or max(1, b_cols)
    ldc = ldc or max(1, N)
    dA, dB = dev(A), dev(B)
    a_rows = A.shape[-2] if A.ndim >= 2 else 1
    b_rows = B.shape[-2] if B.ndim >= 2 else 1
    sA = a_rows * lda
    sB = b_rows * ldb
    sC = M * ldc
    dC = torch.full((batch, M, ldc), float("nan"), dtype=torch.float32, device="cuda")
    dbias = dev(bias) if bias is not None else None
    daux = None
    if aux is not None:
        aux_p = np.zeros((batch, M, ldc), np.float32)
        aux_p[:, :, :N] = aux.reshape(batch, M, N)
        daux = dev(aux_p)
    ptrs = (dbias.data_ptr() if dbias is not None else None,
            daux.data_ptr() if daux is not None else None)
    if workspace is None:
        capi.sgemm_ex_select(ta, tb, M, N, K, dA.data_ptr(), lda, sA, dB.data_ptr(), ldb, sB,
                             dC.data_ptr(), ldc, sC, batch, *ptrs, epilogue, kernel, stream())
    else:
        assert kernel == capi.KERNEL_AUTO
        ws = torch.full((max(1, workspace // 4),), float("nan"), dtype=torch.float32,
                        device="cuda")
        capi.sgemm_ex_ws(ta, tb, M, N, K, dA.data_ptr(), lda, sA, dB.data_ptr(), ldb, sB,
                         dC.data_ptr(), ldc, sC, batch, *ptrs, epilogue, ws.data_ptr(),
                         workspace, stream())
    return host(dC)[:, :, :N]


def ref64(ta, tb, A, B, M, N, K, batch=1, bias=None, aux=None, epilogue=0):
    """fp64 product and |A||B| (+|bias|) with numpy BLAS, the epilogue applied in fp64.

    Same definition as oracle.sgemm_ex_f64 (pinned equal in tests/test_oracle.py),
    but fast enough for the full-size configurations.
    """
    A64 = A.reshape(batch, *A.shape[-2:]).astype(np.float64)
    B64 = B.reshape(batch, *B.shape[-2:]).astype(np.float64)
    opA = np.swapaxes(A64, 1, 2) if ta else A64
    opB = np.swapaxes(B64, 1, 2) if tb else B64
    c = opA @ opB
    s = np.abs(opA) @ np.abs(opB)
    if epilogue in (1, 2):
        c = c + bias.astype(np.float64)
        s = s + np.abs(bias.astype(np.float64))
    if epilogue in (2, 3):
        c = np.where(c > 0, c, 0.0)
    if epilogue == 4:
        c = np.where(aux.reshape(batch, M, N) > 0, c, 0.0)
    return c, s


def check_gemm(c_gpu, ta, tb, A, B, M, N, K, batch=1, bias=None, aux=None, epilogue=0,
               fp32_oracle=None):
    """Compare with fp64 (elementwise bound + normwise 1e-4) and the fp32 oracle loop."""
    assert np.all(np.isfinite(c_gpu)), "unwritten or non-finite output"
    c64, s64 = ref64(ta, tb, A, B, M, N, K, batch=batch, bias=bias, aux=aux,
                     epilogue=epilogue)
    if fp32_oracle is None:
        fp32_oracle = batch * M * N * K <= 64 * 1024 * 1024
    tol = oracle.gemm_tolerance(s64, K)
    err64 = np.abs(c_gpu.astype(np.float64) - c64)
    worst = float(np.max(err64 / tol)) if err64.size else 0.0
    assert np.all(err64 <= tol), f"elementwise bound exceeded: max err/tol = {worst:.3f}"
    scale = float(np.max(np.abs(c64))) if c64.size else 0.0
    if scale > 0:
        assert float(np.max(err64)) / scale <= 1e-4
    if fp32_oracle:
        c32 = oracle.sgemm_ex(ta, tb, A, B, M, N, K, batch=batch, bias=bias, aux=aux,
                              epilogue=epilogue)
        err32 = np.abs(c_gpu.astype(np.float64) - c32.astype(np.float64))
        assert np.all(err32 <= 2.0 * tol), "fp32 oracle disagrees beyond 2x bound"
    return worst
