"""fdl_sgemm_ex_noalloc (the library's static per-GPU scratch in place of a
workspace argument) against fdl_sgemm_ex_ws, through the C-ABI.

Both run the same kernels in the same order, so the bar is bit-for-bit
equality, plus the GEMM parity bound against fp64.  Two calls in a row, the
second smaller, show that the scratch left by one call does not leak into the
next.
"""
import numpy as np
import pytest

import fast_dl_amd.capi as capi
from tests.conftest import rng
from tests.gpu_helpers import check_gemm, dev, host, say, stream

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20


def _gemm(entry, M, N, K, A, B, bias, epi):
    import torch

    dA, dB, dbias = dev(A), dev(B), dev(bias)
    dC = torch.full((M, N), float("nan"), device="cuda")
    args = (0, 0, M, N, K, dA.data_ptr(), K, 0, dB.data_ptr(), N, 0, dC.data_ptr(), N, 0, 1,
            dbias.data_ptr(), None, epi)
    if entry == "noalloc":
        capi.sgemm_ex_noalloc(*args, stream())
    elif entry == "ws":
        nbytes = capi.workspace_size(0, 0, M, N, K)
        ws = torch.full((max(1, nbytes // 4),), float("nan"), device="cuda")
        capi.sgemm_ex_ws(*args, ws.data_ptr(), nbytes, stream())
    else:
        capi.sgemm_ex(*args, stream())
    return host(dC)


def test_noalloc_matches_workspace_entry(device):
    # the largest problem the scratch holds (C5a at M = 8), then a smaller one
    for M, N, K in [(8, 4096, 4096), (1, 1024, 4096)]:
        need = capi.workspace_size(0, 0, M, N, K)
        assert 0 < need <= SCRATCH_BYTES
        g = rng(M * 1000 + N)
        A = g.standard_normal((M, K), dtype=np.float32)
        B = g.standard_normal((K, N), dtype=np.float32)
        bias = (g.standard_normal(N) * 0.1).astype(np.float32)
        say(f"sgemm_noalloc M={M} N={N} K={K} (scratch {need} bytes)")
        c_na = _gemm("noalloc", M, N, K, A, B, bias, capi.EPILOGUE_BIAS_RELU)
        c_ws = _gemm("ws", M, N, K, A, B, bias, capi.EPILOGUE_BIAS_RELU)
        assert np.array_equal(c_na, c_ws)
        check_gemm(c_na[None], 0, 0, A[None], B[None], M, N, K, bias=bias,
                   epilogue=capi.EPILOGUE_BIAS_RELU, fp32_oracle=False)


def test_noalloc_without_scratch_and_beyond_it(device):
    # a problem that needs no scratch runs as fdl_sgemm_ex
    g = rng(7)
    M = N = K = 256
    A = g.standard_normal((M, K), dtype=np.float32)
    B = g.standard_normal((K, N), dtype=np.float32)
    bias = np.zeros(N, np.float32)
    assert capi.workspace_size(0, 0, M, N, K) == 0
    say("sgemm_noalloc 256^3 (no scratch)")
    assert np.array_equal(_gemm("noalloc", M, N, K, A, B, bias, 0),
                          _gemm("plain", M, N, K, A, B, bias, 0))
    # one that needs more than the scratch holds is refused before any launch
    assert capi.workspace_size(0, 0, 8, 43776, 4096) > SCRATCH_BYTES
    # null operands: the scratch-size refusal comes first, and were that check
    # ever to regress, the null-pointer check still refuses before any launch
    status = capi.raw_call("fdl_sgemm_ex_noalloc", 0, 0, 8, 43776, 4096, None, 4096, 0,
                           None, 43776, 0, None, 43776, 0, 1, None, None, 0, None)
    assert status == -1
    assert "bytes of scratch" in capi.last_error()
