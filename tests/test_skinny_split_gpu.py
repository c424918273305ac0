"""GPU parity of the skinny family's K-split form (fdl_sgemm_ex_ws).

Same bar as the other GEMM parity tests: every element within
c0*(sqrt(K)+2)*FLT_EPSILON*(|A||B| + |bias|) of the fp64 product (c0 = 2),
normwise relative error <= 1e-4, within twice that bound of the fp32
restatement of the reference loop where it runs in seconds, and bit for bit
on integer-valued inputs (every partial sum exact in fp32).
"""
import numpy as np
import pytest

import fast_dl_amd.capi as capi
from tests.conftest import rng
from tests.gpu_helpers import check_gemm, dev, gpu_sgemm, host, operands, say, stream

pytestmark = pytest.mark.gpu

# (M, N, K, transA, epilogue): full bands and a part band, K slices of equal
# and unequal length, 8 to 64 slices, M of every register-tile size (1, 2, 4,
# 8) and between, and two plans whose slices would start a multiple of 4 MiB
# of B apart and take 8 more rows each instead (the last slice shorter).
CASES = [
    (8, 4096, 8192, 0, capi.EPILOGUE_BIAS_RELU),
    (8, 16384, 1024, 0, capi.EPILOGUE_BIAS),
    (1, 4096, 4096, 0, capi.EPILOGUE_BIAS_RELU),
    (8, 4096, 4096, 0, capi.EPILOGUE_BIAS_RELU),
    (3, 1024, 4096, 1, capi.EPILOGUE_NONE),
    (2, 260, 16384, 0, capi.EPILOGUE_BIAS),
    (7, 8192, 1100, 1, capi.EPILOGUE_RELU),
    (5, 2048, 4099, 0, capi.EPILOGUE_RELU_GRAD),
    (4, 100, 100000, 0, capi.EPILOGUE_BIAS_RELU),
    (6, 16388, 512, 0, capi.EPILOGUE_NONE),
]


def _inputs(g, M, N, K, ta, epi, dist="normal"):
    A, B = operands(g, ta, 0, M, N, K, 1, dist=dist)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    aux = g.standard_normal((1, M, N)).astype(np.float32) if epi == capi.EPILOGUE_RELU_GRAD else None
    return A, B, bias, aux


@pytest.mark.parametrize("M,N,K,ta,epi", CASES)
def test_split_matches_fp64(device, M, N, K, ta, epi):
    ws = capi.workspace_size(ta, 0, M, N, K)
    assert ws > 0, "the case must take the K split"
    g = rng(M * 7919 + N + K)
    A, B, bias, aux = _inputs(g, M, N, K, ta, epi)
    say(f"skinny split M={M} N={N} K={K} ta={ta} epi={epi} ws={ws}")
    c = gpu_sgemm(ta, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi, workspace=ws)
    check_gemm(c, ta, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi,
               fp32_oracle=M * N * K <= 16 * 1024 * 1024)
    # repeatable bit for bit (fixed slice and wave order)
    c2 = gpu_sgemm(ta, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi, workspace=ws)
    assert np.array_equal(c, c2)


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (8, 1024, 8192), (3, 516, 20000),
                                   (8, 4096, 8192)])
def test_split_exact_on_integers(device, M, N, K):
    # integer operands in [-4, 4]: |partial sums| <= 16 K < 2^24, so every order is exact
    g = rng(17 + M + N)
    A, B = operands(g, 0, 0, M, N, K, 1, dist="int")
    ws = capi.workspace_size(0, 0, M, N, K)
    assert ws > 0
    say(f"skinny split integers M={M} N={N} K={K}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, workspace=ws)
    exact = (A[0].astype(np.int64) @ B[0].astype(np.int64)).astype(np.float32)
    assert np.array_equal(c[0], exact)


def test_small_workspace_runs_single_pass(device):
    # less than fdl_sgemm_workspace_size: exactly fdl_sgemm_ex (the strip kernel)
    M, N, K = 8, 4096, 4096
    g = rng(99)
    A, B, bias, _ = _inputs(g, M, N, K, 0, capi.EPILOGUE_BIAS)
    ws = capi.workspace_size(0, 0, M, N, K)
    say("skinny split: workspace one float short")
    c_small = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS,
                        workspace=ws - 4)
    c_plain = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS)
    assert np.array_equal(c_small, c_plain)
    c_split = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS,
                        workspace=ws)
    assert not np.array_equal(c_split, c_plain)  # a different summation order
    check_gemm(c_split, 0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS,
               fp32_oracle=False)


def test_workspace_ignored_elsewhere(device):
    # problems outside the skinny family, batched problems and transposed B
    # run exactly as fdl_sgemm_ex and leave the workspace untouched
    import torch

    g = rng(5)
    for (ta, tb, M, N, K, batch) in [(0, 0, 256, 256, 256, 1), (0, 0, 4, 4096, 1024, 2),
                                     (0, 1, 4, 4096, 1024, 1)]:
        assert capi.workspace_size(ta, tb, M, N, K, batch) == 0
        A, B = operands(g, ta, tb, M, N, K, batch)
        say(f"workspace ignored ta={ta} tb={tb} M={M} N={N} K={K} batch={batch}")
        ref = gpu_sgemm(ta, tb, A, B, M, N, K, batch=batch)
        dA, dB = dev(A), dev(B)
        dC = torch.full((batch, M, N), float("nan"), device="cuda")
        ws = torch.full((1 << 20,), float("nan"), device="cuda")
        capi.sgemm_ex_ws(ta, tb, M, N, K, dA.data_ptr(), K if not ta else M, A[0].size,
                         dB.data_ptr(), N if not tb else K, B[0].size, dC.data_ptr(), N, M * N,
                         batch, None, None, 0, ws.data_ptr(), 4 << 20, stream())
        assert np.array_equal(host(dC), ref)
        assert torch.isnan(ws).all().item()


def test_misaligned_workspace_rejected(device):
    import torch

    M, N, K = 1, 4096, 4096
    dA = torch.zeros((M, K), device="cuda")
    dB = torch.zeros((K, N), device="cuda")
    dC = torch.zeros((M, N), device="cuda")
    ws = torch.zeros((1 << 18,), device="cuda")
    with pytest.raises(capi.FdlError, match="16-byte aligned"):
        capi.sgemm_ex_ws(0, 0, M, N, K, dA.data_ptr(), K, 0, dB.data_ptr(), N, 0, dC.data_ptr(),
                         N, 0, 1, None, None, 0, ws.data_ptr() + 4, 1 << 20, stream())
