"""GPU parity of the four-wave tiles with hand-scheduled K loops (sgemm.hip's
CfgDma256W4, CfgDma128W4 and CfgDma64W4, the loops in dma_loops.inc, one per
layout), which run the problems FDL_KERNEL_DMA256, FDL_KERNEL_DMA128W8 and
(at most one block per CU) FDL_KERNEL_DMA64 take with K >= 256.

Each output adds the same products in the same order whatever the layout, so
the four layouts of one product must agree bit for bit; the 256x256 and
128x128 tiles also agree with their eight-wave forms below K = 256 (the
64x64 tile's other forms split K over two sets of waves, another order).  K values
cover every way the asm loops hand over to the compiled loop: whole groups of
three steady K-tiles, then zero, one or two more steady tiles and the checked
last tiles, with and without a partial last K-tile."""
import zlib

import numpy as np
import pytest

import fast_dl_amd.capi as capi
from tests.gpu_helpers import check_gemm, dev, gpu_sgemm, host, operands, say, stream

pytestmark = pytest.mark.gpu

FAMS = [capi.KERNEL_DMA256, capi.KERNEL_DMA128W8, capi.KERNEL_DMA64]
# K-tiles of 16 (256x256 tile): 16..21 K-tiles give (K-tiles - 2) % 3 = 2, 0,
# 1, 2, 0, 1; K-tiles of 32 (128x128 tile): 8, 9 (partial), 9, 10 (partial),
# 10, 11 (partial).  1000 and 4100 end in a partial K-tile; 252 stays below
# the loops' threshold.
KS = [256, 272, 288, 304, 320, 336, 1000, 4100, 252]


def _rng(*key):
    # crc32 of the key's text, not hash(): string hashing changes per process
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


@pytest.mark.parametrize("fam", FAMS)
@pytest.mark.parametrize("K", KS)
def test_w4_layouts_agree_bitwise(device, fam, K):
    M, N = 520, 300
    g = _rng("w4", K)
    A, B = operands(g, 0, 0, M, N, K, 1)
    At = np.ascontiguousarray(np.swapaxes(A, 1, 2))
    Bt = np.ascontiguousarray(np.swapaxes(B, 1, 2))
    say(f"fam={fam} NN/NT/TN/TT, K={K}")
    c_nn = gpu_sgemm(0, 0, A, B, M, N, K, kernel=fam)
    check_gemm(c_nn, 0, 0, A, B, M, N, K, fp32_oracle=False)
    for ta, tb, a, b in ((0, 1, A, Bt), (1, 0, At, B), (1, 1, At, Bt)):
        c = gpu_sgemm(ta, tb, a, b, M, N, K, kernel=fam)
        assert np.array_equal(c_nn.view(np.uint32), c.view(np.uint32)), (ta, tb)


@pytest.mark.parametrize("fam", FAMS[:2])
def test_w4_matches_eight_wave_form_bitwise(device, fam):
    """The same product with K = 252 (the eight-wave form) and K = 256 whose
    last four k rows of A are zero (the four-wave form): equal bit for bit,
    since the zero products add exactly."""
    M, N = 520, 300
    g = _rng("w4vs8", fam)
    A, B = operands(g, 0, 0, M, N, 256, 1)
    A[:, :, 252:] = 0.0
    say(f"fam={fam} K=252 eight-wave vs K=256 four-wave")
    c8 = gpu_sgemm(0, 0, np.ascontiguousarray(A[:, :, :252]),
                   np.ascontiguousarray(B[:, :252, :]), M, N, 252, kernel=fam)
    c4 = gpu_sgemm(0, 0, A, B, M, N, 256, kernel=fam)
    assert np.array_equal(c8.view(np.uint32), c4.view(np.uint32))


@pytest.mark.parametrize("fam", FAMS)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("epi", [capi.EPILOGUE_NONE, capi.EPILOGUE_BIAS, capi.EPILOGUE_BIAS_RELU,
                                 capi.EPILOGUE_RELU])
def test_w4_epilogues_and_batch(device, fam, ta, tb, epi):
    M, N, K, batch = 300, 520, 304, 3
    g = _rng("w4e", epi, ta, tb)
    A, B = operands(g, ta, tb, M, N, K, batch)
    bias = g.standard_normal(N).astype(np.float32)
    say(f"fam={fam} four-wave ta={ta} tb={tb} epilogue {epi}, batch {batch}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, batch=batch, bias=bias, epilogue=epi, kernel=fam)
    check_gemm(c, ta, tb, A, B, M, N, K, batch=batch, bias=bias, epilogue=epi, fp32_oracle=False)


@pytest.mark.parametrize("fam", FAMS)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_w4_integer_inputs_exact(device, fam, ta, tb):
    # Small integers: every partial sum is exact in fp32, so any order agrees.
    M, N, K = 512, 512, 1024
    A, B = operands(_rng("w4i", ta, tb), ta, tb, M, N, K, 1, dist="int")
    say(f"fam={fam} four-wave integer inputs ta={ta} tb={tb}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)
    a = A[0].T if ta else A[0]
    b = B[0].T if tb else B[0]
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(c[0].astype(np.float64), exact)


@pytest.mark.parametrize("fam", FAMS)
def test_w4_padded_leading_dimensions(device, fam):
    M, N, K = 260, 520, 512
    g = _rng("w4p")
    A, B = operands(g, 0, 0, M, N, K, 1)
    Ap = np.zeros((1, M, K + 36), np.float32)
    Ap[:, :, :K] = A
    Bp = np.zeros((1, K, N + 12), np.float32)
    Bp[:, :, :N] = B
    say(f"fam={fam} four-wave padded lda/ldb/ldc")
    c = gpu_sgemm(0, 0, Ap, Bp, M, N, K, kernel=fam, lda=K + 36, ldb=N + 12, ldc=N + 8)
    check_gemm(c, 0, 0, A, B, M, N, K)


@pytest.mark.parametrize("fam", FAMS)
def test_w4_operand_past_two_gib_falls_back(device, fam):
    """A spans more than 2 GiB (130 rows at lda = 2^22, the largest leading
    dimension the direct-to-LDS kernels take): the four-wave loops' 32-bit
    copy offsets are not used, the eight-wave kernel runs, and the result is
    still right."""
    import torch

    M, N, K = 130, 256, 512
    lda = 1 << 22
    g = _rng("w4big")
    A, B = operands(g, 0, 0, M, N, K, 1)
    say(f"fam={fam} with a 2.2 GB A (lda 2^22)")
    dA = torch.zeros((M, lda), dtype=torch.float32, device="cuda")
    dA[:, :K] = torch.from_numpy(A[0]).cuda()
    dB = dev(B)
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    capi.sgemm_ex_select(0, 0, M, N, K, dA.data_ptr(), lda, M * lda, dB.data_ptr(), N, K * N,
                         dC.data_ptr(), N, M * N, 1, None, None, 0, fam, stream())
    c = host(dC)[None]
    del dA
    check_gemm(c, 0, 0, A, B, M, N, K, fp32_oracle=False)


def test_leading_dimension_past_dma_limit(device):
    """lda above 2^22 floats: forcing a direct-to-LDS kernel is refused
    (FDL_ERROR_NOT_SUPPORTED) and the automatic choice takes another kernel."""
    import torch

    M, N, K = 8 * 64, 512, 256
    lda = (1 << 22) + 4
    g = _rng("ldbig")
    A, B = operands(g, 0, 0, M, N, K, 1)
    say("lda 2^22 + 4: forced dma256 refused, auto correct")
    dA = torch.zeros((M, lda), dtype=torch.float32, device="cuda")
    dA[:, :K] = torch.from_numpy(A[0]).cuda()
    dB = dev(B)
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    args = (0, 0, M, N, K, dA.data_ptr(), lda, M * lda, dB.data_ptr(), N, K * N,
            dC.data_ptr(), N, M * N, 1, None, None, 0)
    with pytest.raises(capi.FdlError) as err:
        capi.sgemm_ex_select(*args, capi.KERNEL_DMA256, stream())
    assert "2^22" in str(err.value)
    capi.sgemm_ex_select(*args, capi.KERNEL_AUTO, stream())
    c = host(dC)[None]
    del dA
    check_gemm(c, 0, 0, A, B, M, N, K, fp32_oracle=False)
