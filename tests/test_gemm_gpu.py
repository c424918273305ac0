"""GPU parity of fdl_sgemm_ex (every kernel family) against the CPU oracle.

Bar: every element within c0*(sqrt(K)+2)*FLT_EPSILON*(|A||B| + |bias|) of the
fp64 twin (c0 = 2), normwise relative error <= 1e-4, and within twice that
bound of the fp32 restatement of the reference loop.  Integer-valued inputs
(exact in fp32) must match bit for bit.
"""
import hashlib

import numpy as np
import pytest

import fast_dl_amd.capi as capi
import oracle
from tests.conftest import rng
from tests.gpu_helpers import check_gemm, dev, gpu_sgemm, host, operands, say, stream

pytestmark = pytest.mark.gpu

FAMILIES = [capi.KERNEL_TILED128, capi.KERNEL_TILED64, capi.KERNEL_SPLITK32,
            capi.KERNEL_TILED256, capi.KERNEL_TILED256X128, capi.KERNEL_TILED128W8,
            capi.KERNEL_SPLITK16]
LAYOUTS = [(0, 0), (0, 1), (1, 0), (1, 1)]


def test_reference_matmul_fixture(device):
    # tests/tensor/matmul_tensor_test.cpp:30-42
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.array([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]], np.float32)
    for fam in FAMILIES + [capi.KERNEL_SKINNY, capi.KERNEL_AUTO]:
        say(f"matmul fixture kernel={fam}")
        c = gpu_sgemm(0, 0, A[None], B[None], 2, 4, 3, kernel=fam)[0]
        assert np.array_equal(c, [[38, 44, 50, 56], [83, 98, 113, 128]])


def test_reference_gemm_entry_point(device):
    # dl::kernels::gemm contract: fdl_gemm(a, b, c, m, n, k) on the null stream.
    import torch

    g = rng(42)
    m, n, k = 64, 96, 80
    a = g.uniform(-1, 1, (m, k)).astype(np.float32)
    b = g.uniform(-1, 1, (k, n)).astype(np.float32)
    da, db = dev(a), dev(b)
    dc = torch.full((m, n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    say("fdl_gemm 64x96x80")
    capi.gemm(da.data_ptr(), db.data_ptr(), dc.data_ptr(), m, n, k)
    c = host(dc)
    cpu = oracle.gemm_cpu(a, b)
    # the reference benchmark's own acceptance rule (gemm_benchmark.cu:50-56)
    assert np.all(np.abs(cpu - c) <= 1e-3 * np.maximum(1.0, np.abs(cpu)))
    check_gemm(c[None], 0, 0, a[None], b[None], m, n, k)


def test_reference_linear_fixture(device):
    # tests/tensor/linear_tensor_test.cpp:38-53 through the fused bias epilogue
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    w = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    b = np.array([0.5, 1.0], np.float32)
    for fam in FAMILIES + [capi.KERNEL_SKINNY]:
        say(f"linear fixture kernel={fam}")
        y = gpu_sgemm(0, 0, x[None], w[None], 2, 2, 3, bias=b, epilogue=capi.EPILOGUE_BIAS,
                      kernel=fam)[0]
        assert np.allclose(y, [[22.5, 29.0], [49.5, 65.0]], atol=1e-4, rtol=0)


SHAPES = [(1, 1, 1), (7, 5, 3), (33, 17, 65), (64, 64, 16), (127, 129, 31),
          (128, 128, 128), (130, 260, 17), (200, 72, 257)]


@pytest.mark.parametrize("fam", FAMILIES)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_layouts_and_edges(device, fam, ta, tb, M, N, K):
    g = rng(hash((M, N, K, ta, tb)) & 0xFFFF)
    A, B = _ops(g, ta, tb, M, N, K, 1)
    say(f"sgemm fam={fam} ta={ta} tb={tb} M={M} N={N} K={K}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)
    check_gemm(c, ta, tb, A, B, M, N, K)


def _ops(g, ta, tb, M, N, K, batch, scale=1.0):
    A = (g.standard_normal((batch, K, M) if ta else (batch, M, K)) * scale).astype(np.float32)
    B = (g.standard_normal((batch, N, K) if tb else (batch, K, N)) * scale).astype(np.float32)
    return A, B


@pytest.mark.parametrize("fam", FAMILIES)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_integer_inputs_bit_exact(device, fam, ta, tb):
    g = rng(99)
    M, N, K = 150, 140, 300
    A = g.integers(-4, 5, (1, K, M) if ta else (1, M, K)).astype(np.float32)
    B = g.integers(-4, 5, (1, N, K) if tb else (1, K, N)).astype(np.float32)
    say(f"integer exact fam={fam} ta={ta} tb={tb}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)[0]
    opA = (A[0].T if ta else A[0]).astype(np.int64)
    opB = (B[0].T if tb else B[0]).astype(np.int64)
    assert np.array_equal(c, (opA @ opB).astype(np.float32))


@pytest.mark.parametrize("fam", FAMILIES + [capi.KERNEL_SKINNY])
@pytest.mark.parametrize("epi", [capi.EPILOGUE_BIAS, capi.EPILOGUE_BIAS_RELU,
                                 capi.EPILOGUE_RELU, capi.EPILOGUE_RELU_GRAD])
def test_epilogues(device, fam, epi):
    g = rng(100 + epi)
    M, N, K = (7, 300, 129) if fam == capi.KERNEL_SKINNY else (150, 90, 77)
    A, B = _ops(g, 0, 0, M, N, K, 1)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    aux = g.standard_normal((1, M, N)).astype(np.float32)
    say(f"epilogue fam={fam} epi={epi}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi, kernel=fam)
    check_gemm(c, 0, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi)


def test_config1_mnist_like(device):
    # M=256, K=784, N=128; A ~ U[0,1), B ~ N(0, sqrt(2/784))
    g = rng(1)
    M, K, N = 256, 784, 128
    A = g.random((1, M, K)).astype(np.float32)
    B = (g.standard_normal((1, K, N)) * np.sqrt(2.0 / 784)).astype(np.float32)
    for fam in FAMILIES + [capi.KERNEL_AUTO]:
        say(f"config1 fam={fam}")
        c = gpu_sgemm(0, 0, A, B, M, N, K, kernel=fam)
        check_gemm(c, 0, 0, A, B, M, N, K)
    gold = np.load(_golden("config1_gemm.npz"))
    assert hashlib.sha256(A.tobytes()).digest() == gold["sha_A"].tobytes()
    assert hashlib.sha256(B.tobytes()).digest() == gold["sha_B"].tobytes()
    c = gpu_sgemm(0, 0, A, B, M, N, K)[0]
    tol = oracle.gemm_tolerance(np.abs(A[0]).astype(np.float64) @ np.abs(B[0]).astype(np.float64), K)
    assert np.all(np.abs(c.astype(np.float64) - gold["C64"]) <= tol)
    assert np.all(np.abs(c - gold["C32"]) <= 2 * tol)


def _golden(name):
    import os

    return os.path.join(os.path.dirname(__file__), "golden", name)


@pytest.mark.parametrize("tb", [0, 1])
def test_config4_batched(device, tb):
    # batch 64 of [128x64].[64x128], N(0, 1/8), NN and NT
    g = rng(4)
    batch, M, K, N = 64, 128, 64, 128
    A, B = _ops(g, 0, tb, M, N, K, batch, scale=np.sqrt(1 / 8))
    for fam in FAMILIES + [capi.KERNEL_DMA64, capi.KERNEL_DMA64S, capi.KERNEL_DMA64U,
                           capi.KERNEL_AUTO]:
        say(f"config4 tb={tb} fam={fam}")
        c = gpu_sgemm(0, tb, A, B, M, N, K, batch=batch, kernel=fam)
        check_gemm(c, 0, tb, A, B, M, N, K, batch=batch, fp32_oracle=(fam == capi.KERNEL_AUTO))


def test_batched_broadcast_and_padded_ld(device):
    import torch

    g = rng(8)
    batch, M, N, K = 3, 70, 50, 40
    lda, ldb, ldc = K + 5, N + 3, N + 7
    A = g.standard_normal((batch, M, lda)).astype(np.float32)
    B = g.standard_normal((1, K, ldb)).astype(np.float32)  # stride 0: shared by all batches
    dA, dB = dev(A), dev(B)
    dC = torch.full((batch, M, ldc), float("nan"), device="cuda")
    for fam in FAMILIES:
        say(f"padded ld / broadcast fam={fam}")
        capi.sgemm_ex_select(0, 0, M, N, K, dA.data_ptr(), lda, M * lda, dB.data_ptr(), ldb, 0,
                             dC.data_ptr(), ldc, M * ldc, batch, None, None, 0, fam, stream())
        c = host(dC)
        assert np.all(np.isnan(c[:, :, N:])), "wrote outside the ldc window"
        Ap = np.ascontiguousarray(A[:, :, :K])
        Bp = np.ascontiguousarray(np.broadcast_to(B[:, :, :N], (batch, K, N)))
        check_gemm(np.ascontiguousarray(c[:, :, :N]), 0, 0, Ap, Bp, M, N, K, batch=batch)


@pytest.mark.parametrize("fam", ["dma64", "dma64s", "splitk16", "splitk32", "skinny"])
def test_batch_stride_beyond_int32(device, fam):
    # These kernels take batch strides as 32-bit arguments; a stride past
    # 2^31 - 1 runs one problem per launch.  A's two problems sit 2^31 + 256
    # floats (8 GiB) apart in one allocation, B is shared.
    import torch

    kernel = {"dma64": capi.KERNEL_DMA64, "dma64s": capi.KERNEL_DMA64S,
              "splitk16": capi.KERNEL_SPLITK16, "splitk32": capi.KERNEL_SPLITK32,
              "skinny": capi.KERNEL_SKINNY}[fam]
    g = rng(9)
    batch, M, N, K = 2, (8 if fam == "skinny" else 64), 64, 64
    A = g.standard_normal((batch, M, K)).astype(np.float32)
    B = g.standard_normal((1, K, N)).astype(np.float32)
    sA = (1 << 31) + 256
    big = torch.empty(sA + M * K, device="cuda")
    big[: M * K] = dev(A[0]).reshape(-1)
    big[sA : sA + M * K] = dev(A[1]).reshape(-1)
    dB = dev(B)
    dC = torch.full((batch, M, N), float("nan"), device="cuda")
    say(f"stride beyond int32 fam={fam}")
    capi.sgemm_ex_select(0, 0, M, N, K, big.data_ptr(), K, sA, dB.data_ptr(), N, 0,
                         dC.data_ptr(), N, M * N, batch, None, None, 0, kernel, stream())
    c = host(dC)
    del big
    torch.cuda.empty_cache()
    check_gemm(c, 0, 0, A, np.ascontiguousarray(np.broadcast_to(B, (batch, K, N))), M, N, K,
               batch=batch)


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_skinny_vs_oracle(device, M):
    g = rng(50 + M)
    N, K = 1000, 700
    A, B = _ops(g, 0, 0, M, N, K, 1)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    for ta in (0, 1):
        Aop = np.ascontiguousarray(np.swapaxes(A, 1, 2)) if ta else A
        say(f"skinny M={M} ta={ta}")
        c = gpu_sgemm(ta, 0, Aop, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU,
                      kernel=capi.KERNEL_SKINNY)
        check_gemm(c, ta, 0, Aop, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU)
    # N not a multiple of 4 takes the scalar column path
    A2, B2 = _ops(g, 0, 0, M, 301, 65, 1)
    say(f"skinny scalar M={M}")
    c = gpu_sgemm(0, 0, A2, B2, M, 301, 65, kernel=capi.KERNEL_SKINNY)
    check_gemm(c, 0, 0, A2, B2, M, 301, 65)


@pytest.mark.parametrize("M", [1, 8])
def test_config5_skinny_full_size(device, M):
    # BASELINE config 5a: M in {1, 8}, K = N = 4096, bias + ReLU, operands N(0,1), bias N(0, 0.1)
    g = rng(5 + M)
    N = K = 4096
    A, B = _ops(g, 0, 0, M, N, K, 1)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    say(f"config5a M={M}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU)
    check_gemm(c, 0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU,
               fp32_oracle=False)


@pytest.mark.parametrize("n", [777, 1000, 1023])
def test_config5_non_tile_multiples(device, n):
    # BASELINE config 5b: M = N = K in {777, 1000, 1023}, bias + ReLU
    g = rng(n)
    A, B = _ops(g, 0, 0, n, n, n, 1)
    bias = (g.standard_normal(n) * 0.1).astype(np.float32)
    for fam in FAMILIES + [capi.KERNEL_DMA64U, capi.KERNEL_DMA96X32U, capi.KERNEL_AUTO]:
        say(f"config5b n={n} fam={fam}")
        c = gpu_sgemm(0, 0, A, B, n, n, n, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU,
                      kernel=fam)
        check_gemm(c, 0, 0, A, B, n, n, n, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU,
                   fp32_oracle=False)


@pytest.mark.parametrize("n", [1024, 2048, 4096, 8192])
def test_config3_square_sampled_rows(device, n):
    # BASELINE config 3 at full size, through the automatic choice (dma256 from 4096):
    # a contiguous 64-row block plus sampled rows against fp64 dot products, as the
    # reference applies its acceptance rule to every shape it runs
    # (tests/benchmarks/gemm/gemm_benchmark.cu:50-56)
    import torch

    g = rng(3000 + n)
    A = g.standard_normal((n, n), dtype=np.float32)
    B = g.standard_normal((n, n), dtype=np.float32)
    say(f"config3 n={n} kernel={capi.KERNEL_NAMES.get(capi.kernel_choice(0, 0, n, n, n))}")
    dA, dB = dev(A), dev(B)
    dC = torch.full((n, n), float("nan"), device="cuda")
    capi.sgemm_ex(0, 0, n, n, n, dA.data_ptr(), n, 0, dB.data_ptr(), n, 0, dC.data_ptr(), n, 0,
                  1, None, None, 0, stream())
    c = host(dC)
    del dA, dB, dC
    assert np.all(np.isfinite(c))
    block = np.arange(n // 2, n // 2 + 64)
    rows = np.unique(np.concatenate([[0, n - 1], g.integers(0, n, 62), block]))
    c64 = A[rows].astype(np.float64) @ B.astype(np.float64)
    s64 = np.abs(A[rows]).astype(np.float64) @ np.abs(B).astype(np.float64)
    assert np.all(np.abs(c[rows] - c64) <= oracle.gemm_tolerance(s64, n))
    # size-independent checks: linearity in B's columns and a checksum of row sums
    ones = np.ones((n,), np.float64)
    row_sums = A.astype(np.float64) @ (B.astype(np.float64) @ ones)
    tol = oracle.gemm_tolerance(np.abs(A).astype(np.float64) @ (np.abs(B).astype(np.float64) @ ones), n)
    assert np.all(np.abs(c.astype(np.float64).sum(1) - row_sums) <= tol * 4)


def test_degenerate_sizes(device):
    import torch

    bias = np.array([0.5, -1.0, 2.0], np.float32)
    dbias = dev(bias)
    dC = torch.full((4, 3), float("nan"), device="cuda")
    say("K == 0 with bias+relu")
    capi.sgemm_ex(0, 0, 4, 3, 0, None, 1, 0, None, 3, 0, dC.data_ptr(), 3, 0, 1,
                  dbias.data_ptr(), None, capi.EPILOGUE_BIAS_RELU, stream())
    assert np.array_equal(host(dC), np.tile(np.maximum(bias, 0), (4, 1)))
    say("M == 0 / N == 0 / batch == 0 are no-ops")
    dC.fill_(7.0)
    for args in [(0, 3, 5, 1), (4, 0, 5, 1), (4, 3, 5, 0)]:
        M, N, K, batch = args
        capi.sgemm_ex(0, 0, M, N, K, dC.data_ptr(), max(K, 1), 0, dC.data_ptr(), max(N, 1), 0,
                      dC.data_ptr(), max(N, 1), 0, batch, None, None, 0, stream())
    assert np.all(host(dC) == 7.0)


def test_kernel_choice_heuristic(device):
    assert capi.kernel_choice(0, 0, 4096, 4096, 4096) == capi.KERNEL_DMA256
    assert capi.kernel_choice(0, 0, 1, 4096, 4096) == capi.KERNEL_SKINNY
    assert capi.kernel_choice(0, 1, 1, 4096, 4096) != capi.KERNEL_SKINNY


# NN problems with 768 < K <= 1024 and 16-byte rows take the splitk16 form
# that stages each wave's K range in LDS (C1 and the MLP forward are such
# problems).  The same operands with a row pitch that is not a multiple of 4
# floats take the register form, whose k order and wave order it keeps.
@pytest.mark.parametrize("M,N,K,batch,epi", [
    (256, 128, 784, 1, capi.EPILOGUE_NONE),
    (256, 256, 784, 1, capi.EPILOGUE_BIAS_RELU),
    (33, 20, 772, 1, capi.EPILOGUE_BIAS),
    (17, 44, 1024, 3, capi.EPILOGUE_RELU),
    (130, 36, 1000, 1, capi.EPILOGUE_RELU_GRAD),
    (16, 16, 788, 2, capi.EPILOGUE_NONE),
])
def test_splitk16_lds_staged(device, M, N, K, batch, epi):
    g = rng(M * 131 + N * 17 + K)
    A, B = operands(g, 0, 0, M, N, K, batch)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    aux = (g.standard_normal((batch, M, N)).astype(np.float32)
           if epi == capi.EPILOGUE_RELU_GRAD else None)
    say(f"splitk16 LDS-staged M={M} N={N} K={K} batch={batch} epi={epi}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, batch=batch, bias=bias, aux=aux, epilogue=epi,
                  kernel=capi.KERNEL_SPLITK16)
    check_gemm(c, 0, 0, A, B, M, N, K, batch=batch, bias=bias, aux=aux, epilogue=epi,
               fp32_oracle=True)
    # the register form on the same values (row pitch K + 1): the same bits
    A_pad = np.zeros((batch, M, K + 1), np.float32)
    A_pad[:, :, :K] = A
    c_reg = gpu_sgemm(0, 0, A_pad, B, M, N, K, batch=batch, bias=bias, aux=aux, epilogue=epi,
                      kernel=capi.KERNEL_SPLITK16, lda=K + 1)
    assert np.array_equal(c, c_reg)
    # integer operands: every order exact
    Ai, Bi = operands(g, 0, 0, M, N, K, batch, dist="int")
    ci = gpu_sgemm(0, 0, Ai, Bi, M, N, K, batch=batch, kernel=capi.KERNEL_SPLITK16)
    exact = np.einsum("bmk,bkn->bmn", Ai.astype(np.int64), Bi.astype(np.int64))
    assert np.array_equal(ci, exact.astype(np.float32))


@pytest.mark.parametrize("wide", ["lda", "ldb"])
def test_splitk16_lds_form_wide_pitch_takes_register_form(device, wide):
    """The LDS-staged split-K16 form addresses its copies with 32-bit offsets, so it takes
    lda < 2^24 and ldb < 2^22; past either, the same problem runs the register form, which
    gives the LDS form's bits.  The wide operand is a strided view of one large
    allocation (2 GB for A, 13 GB for B), only its used elements written."""
    import torch

    M, N, K = 32, 16, 800
    g = rng(4243 if wide == "lda" else 4244)
    A, B = operands(g, 0, 0, M, N, K, 1)
    bias = (g.standard_normal(N) * 0.1).astype(np.float32)
    say(f"splitk16 with {wide} past the LDS form's offsets, M={M} N={N} K={K}")
    c_lds = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU,
                      kernel=capi.KERNEL_SPLITK16)
    lda, ldb = K, N
    if wide == "lda":
        lda = 1 << 24
        big = torch.empty((M - 1) * lda + K, dtype=torch.float32, device="cuda")
        torch.as_strided(big, (M, K), (lda, 1)).copy_(torch.from_numpy(A[0]).cuda())
        dA, dB = big, torch.from_numpy(B[0]).cuda()
    else:
        ldb = 1 << 22
        big = torch.empty((K - 1) * ldb + N, dtype=torch.float32, device="cuda")
        torch.as_strided(big, (K, N), (ldb, 1)).copy_(torch.from_numpy(B[0]).cuda())
        dA, dB = torch.from_numpy(A[0]).cuda(), big
    dbias = torch.from_numpy(bias).cuda()
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    capi.sgemm_ex_select(0, 0, M, N, K, dA.data_ptr(), lda, 0, dB.data_ptr(), ldb, 0,
                         dC.data_ptr(), N, 0, 1, dbias.data_ptr(), None,
                         capi.EPILOGUE_BIAS_RELU, capi.KERNEL_SPLITK16, stream())
    c_wide = host(dC).reshape(1, M, N)
    del big
    check_gemm(c_wide, 0, 0, A, B, M, N, K, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU)
    assert np.array_equal(c_wide, c_lds)
