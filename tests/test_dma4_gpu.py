"""GPU parity of the 4-byte-copy direct-to-LDS kernels (FDL_KERNEL_DMA64U,
FDL_KERNEL_DMA96X32U,
FDL_KERNEL_DMA128W8U) on the problems the 16-byte ones refuse: any K (partial
last K-tile of any length), odd M and N, odd leading dimensions and batch
strides, operands one float off a 16-byte boundary; with every epilogue; and
the automatic choice on odd cubes (C5b 777^3 and 1023^3)."""
import numpy as np
import pytest

import fast_dl_amd.capi as capi
from tests.gpu_helpers import check_gemm, dev, gpu_sgemm, host, operands, say, stream

pytestmark = pytest.mark.gpu

DMA4 = [capi.KERNEL_DMA64U, capi.KERNEL_DMA128W8U, capi.KERNEL_DMA96X32U]
LAYOUTS = [(0, 0), (0, 1), (1, 0), (1, 1)]
ODD = [(1, 1, 1), (3, 5, 7), (65, 63, 129), (130, 258, 67), (200, 136, 1023), (257, 129, 65)]


def _rng(*key):
    return np.random.default_rng(abs(hash(key)) & 0xFFFFFFFF)


@pytest.mark.parametrize("fam", DMA4)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("M,N,K", ODD)
def test_dma4_odd_shapes(device, fam, ta, tb, M, N, K):
    A, B = operands(_rng(M, N, K, ta, tb, fam), ta, tb, M, N, K, 1)
    say(f"dma4 fam={fam} ta={ta} tb={tb} M={M} N={N} K={K}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)
    check_gemm(c, ta, tb, A, B, M, N, K)


@pytest.mark.parametrize("fam", DMA4)
@pytest.mark.parametrize("K", [1, 2, 3, 5, 63, 65, 127, 129, 191, 193, 320])
def test_dma4_k_tails(device, fam, K):
    # 1 to 5 K-tiles of 64 with every kind of partial last tile.
    M, N = 96, 70
    A, B = operands(_rng(K, fam), 0, 0, M, N, K, 1, dist="int")
    say(f"dma4 K tail fam={fam} K={K}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, kernel=fam)
    check_gemm(c, 0, 0, A, B, M, N, K)
    # Small integers: every product and partial sum is exact in fp32.
    ref = np.einsum("bmk,bkn->bmn", A.astype(np.float64), B.astype(np.float64))
    assert np.array_equal(c, ref.astype(np.float32))


@pytest.mark.parametrize("fam", DMA4)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_dma4_misaligned_padded_batched(device, fam, ta, tb):
    # Operands one and three floats past a 16-byte boundary, leading
    # dimensions and batch strides that are not multiples of 4.
    import torch

    M, N, K, batch = 131, 97, 150, 3
    A, B = operands(_rng(ta, tb, fam, 5), ta, tb, M, N, K, batch)
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    lda, ldb, ldc = a_cols + 3, b_cols + 1, N + 5
    sA, sB, sC = a_rows * lda + 7, b_rows * ldb + 5, M * ldc + 3
    dA = torch.zeros(1 + batch * sA, device="cuda")
    dB = torch.zeros(3 + batch * sB, device="cuda")
    dC = torch.full((batch * sC,), float("nan"), device="cuda")
    for z in range(batch):
        va = dA[1 + z * sA: 1 + z * sA + a_rows * lda].view(a_rows, lda)
        va[:, :a_cols] = dev(A[z])
        vb = dB[3 + z * sB: 3 + z * sB + b_rows * ldb].view(b_rows, ldb)
        vb[:, :b_cols] = dev(B[z])
    say(f"dma4 misaligned padded batched fam={fam} ta={ta} tb={tb}")
    capi.sgemm_ex_select(ta, tb, M, N, K, dA.data_ptr() + 4, lda, sA, dB.data_ptr() + 12, ldb,
                         sB, dC.data_ptr(), ldc, sC, batch, None, None, 0, fam, stream())
    c = host(dC)
    got = np.stack([c[z * sC: z * sC + M * ldc].reshape(M, ldc)[:, :N] for z in range(batch)])
    check_gemm(got, ta, tb, A, B, M, N, K, batch=batch)


@pytest.mark.parametrize("fam", DMA4)
@pytest.mark.parametrize("epi", [capi.EPILOGUE_BIAS, capi.EPILOGUE_BIAS_RELU,
                                 capi.EPILOGUE_RELU, capi.EPILOGUE_RELU_GRAD])
def test_dma4_epilogues(device, fam, epi):
    M, N, K = 133, 77, 201
    g = _rng(epi, fam, 9)
    A, B = operands(g, 0, 0, M, N, K, 1)
    bias = g.standard_normal(N).astype(np.float32)
    aux = g.standard_normal((1, M, N)).astype(np.float32)
    say(f"dma4 epilogue fam={fam} epi={epi}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi, kernel=fam)
    check_gemm(c, 0, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi)


@pytest.mark.parametrize("n,fam", [(777, capi.KERNEL_DMA96X32U), (1023, capi.KERNEL_DMA64U)])
def test_auto_odd_cubes(device, n, fam):
    # C5b's odd cubes go to the 4-byte-copy tiles, with the fused bias+ReLU
    # epilogue: 777^3 to the 96x32 tile (225 tiles fill the GPU where 169
    # 64x64 ones do not), 1023^3 to the 64x64 one.
    assert capi.kernel_choice(0, 0, n, n, n) == fam
    g = _rng(n, 3)
    A, B = operands(g, 0, 0, n, n, n, 1)
    bias = g.standard_normal(n).astype(np.float32)
    say(f"auto odd cube {n}^3 bias+relu")
    c = gpu_sgemm(0, 0, A, B, n, n, n, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU)
    check_gemm(c, 0, 0, A, B, n, n, n, bias=bias, epilogue=capi.EPILOGUE_BIAS_RELU,
               fp32_oracle=False)
