"""GPU parity of the direct-to-LDS kernels (FDL_KERNEL_DMA256 and
FDL_KERNEL_DMA64S, K-tile 16; FDL_KERNEL_DMA128, K-tile 32; FDL_KERNEL_DMA64
and FDL_KERNEL_DMA128W8, K-tile 64) and of their dispatch rules: they run where K is a multiple of 4 (a partial last K-tile is
clamped and masked) and both operands are 16-byte vectorisable, refuse other
problems with FDL_ERROR_NOT_SUPPORTED when forced, and the automatic choice
falls back to the register-staged kernel with the same tile for misaligned
pointers."""
import numpy as np
import pytest

import fast_dl_amd.capi as capi
from tests.gpu_helpers import check_gemm, dev, gpu_sgemm, host, operands, say, stream

pytestmark = pytest.mark.gpu

DMA = capi.KERNEL_DMA256
DMAS16 = [(capi.KERNEL_DMA256, 16), (capi.KERNEL_DMA128, 32), (capi.KERNEL_DMA64, 64),
          (capi.KERNEL_DMA128W8, 64), (capi.KERNEL_DMA64S, 16)]
# The 4-byte-copy twins run every aligned case too (their own odd-shape cases
# are in test_dma4_gpu.py).
DMAS = DMAS16 + [(capi.KERNEL_DMA64U, 64), (capi.KERNEL_DMA128W8U, 64),
                 (capi.KERNEL_DMA96X32U, 64)]
LAYOUTS = [(0, 0), (0, 1), (1, 0), (1, 1)]
# M and N multiples of 4 (either may be the contiguous extent), ragged against
# the tiles; K in K-tiles (16 or 32 each) covering 1, 2, 3 and many K-tiles.
# (1088, 1040) is 289 blocks of 64x64: more than one per CU, so the 64x64
# configs take their two-stage form there and the three-stage one elsewhere.
SHAPES = [(4, 4, 1), (256, 256, 2), (260, 300, 3), (516, 260, 17), (64, 1000, 6),
          (768, 512, 64), (1088, 1040, 5)]


def _rng(*key):
    return np.random.default_rng(abs(hash(key)) & 0xFFFFFFFF)


@pytest.mark.parametrize("fam,bk", DMAS)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("M,N,kt", SHAPES)
def test_dma_layouts_and_edges(device, fam, bk, ta, tb, M, N, kt):
    K = kt * bk
    A, B = operands(_rng(M, N, K, ta, tb), ta, tb, M, N, K, 1)
    say(f"dma fam={fam} ta={ta} tb={tb} M={M} N={N} K={K}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)
    check_gemm(c, ta, tb, A, B, M, N, K)


@pytest.mark.parametrize("fam,bk", DMAS)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_dma_integer_inputs_bit_exact(device, fam, bk, ta, tb):
    M, N, K = 300, 260, 416
    A, B = operands(_rng(7, ta, tb), ta, tb, M, N, K, 1, dist="int")
    say(f"dma integer exact fam={fam} ta={ta} tb={tb}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)[0]
    opA = (A[0].T if ta else A[0]).astype(np.int64)
    opB = (B[0].T if tb else B[0]).astype(np.int64)
    assert np.array_equal(c, (opA @ opB).astype(np.float32))


@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("K", [16, 32, 48, 64, 4, 28, 60])
def test_dma64s_short_k_bit_exact(device, ta, tb, K):
    # K <= 64 in whole 16-deep K-tiles (1 to 4) runs the straight-line form
    # with every K-tile copied up front; a partial last tile (4, 28, 60) runs
    # the loop.  Small integers: every product and partial sum is exact.
    M, N = 200, 136
    A, B = operands(_rng(19, K, ta, tb), ta, tb, M, N, K, 2, dist="int")
    say(f"dma64s short K={K} ta={ta} tb={tb}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, batch=2, kernel=capi.KERNEL_DMA64S)
    for z in range(2):
        opA = (A[z].T if ta else A[z]).astype(np.int64)
        opB = (B[z].T if tb else B[z]).astype(np.int64)
        assert np.array_equal(c[z], (opA @ opB).astype(np.float32)), f"batch {z}"


@pytest.mark.parametrize("fam,bk", DMAS)
@pytest.mark.parametrize("epi", [capi.EPILOGUE_BIAS, capi.EPILOGUE_BIAS_RELU,
                                 capi.EPILOGUE_RELU, capi.EPILOGUE_RELU_GRAD])
def test_dma_epilogues(device, fam, bk, epi):
    M, N, K = 520, 264, 160
    g = _rng(11, epi)
    A, B = operands(g, 0, 0, M, N, K, 1)
    bias = (g.standard_normal(N) * 0.5).astype(np.float32)
    aux = g.standard_normal((M, N)).astype(np.float32)
    say(f"dma epilogue fam={fam} epi={epi}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi, kernel=fam)
    check_gemm(c, 0, 0, A, B, M, N, K, bias=bias, aux=aux, epilogue=epi)


@pytest.mark.parametrize("fam,bk", DMAS)
def test_dma_batched_and_padded_ld(device, fam, bk):
    M, N, K, batch = 260, 264, 64, 3
    A, B = operands(_rng(13), 0, 1, M, N, K, batch)
    say(f"dma batched NT, padded lda/ldb/ldc fam={fam}")
    # lda/ldb padded to the next multiple of 4 beyond K, ldc beyond N
    lda, ldb, ldc = K + 8, K + 4, N + 12
    Ap = np.zeros((batch, M, lda), np.float32)
    Ap[:, :, :K] = A
    Bp = np.zeros((batch, N, ldb), np.float32)
    Bp[:, :, :K] = B
    c = gpu_sgemm(0, 1, Ap, Bp, M, N, K, batch=batch, kernel=fam, lda=lda, ldb=ldb, ldc=ldc)
    check_gemm(c, 0, 1, A, B, M, N, K, batch=batch)


@pytest.mark.parametrize("fam,bk", DMAS)
@pytest.mark.parametrize("batch", [2, 8, 13, 64])
@pytest.mark.parametrize("tb", [0, 1])
def test_dma_flat_batch_grid(device, fam, bk, batch, tb):
    # Problems of at most 64 tiles each run on a 1-D grid of batch x tiles
    # blocks, renumbered so each XCD owns whole batches when the block count
    # is a multiple of 8 (batch 8 and 64 here; 2 and 13 keep the plain order).
    # A broadcast B (batch stride 0) and padded leading dimensions check the
    # per-batch offsets; C is pre-filled with NaN to catch unwritten tiles.
    import torch

    M, N, K = 136, 100, 48
    g = _rng(31, batch, tb, fam)
    lda, ldb, ldc = K + 4, (K if tb else N) + 8, N + 4
    A = g.standard_normal((batch, M, lda)).astype(np.float32)
    B = g.standard_normal((1, N if tb else K, ldb)).astype(np.float32)
    dA, dB = dev(A), dev(B)
    dC = torch.full((batch, M, ldc), float("nan"), device="cuda")
    say(f"dma flat batch fam={fam} batch={batch} tb={tb}")
    capi.sgemm_ex_select(0, tb, M, N, K, dA.data_ptr(), lda, M * lda, dB.data_ptr(), ldb, 0,
                         dC.data_ptr(), ldc, M * ldc, batch, None, None, 0, fam, stream())
    c = host(dC)
    assert np.all(np.isnan(c[:, :, N:])), "wrote outside the ldc window"
    Ap = np.ascontiguousarray(A[:, :, :K])
    Bv = B[:, :, :K] if tb else B[:, :, :N]
    Bp = np.ascontiguousarray(np.broadcast_to(Bv, (batch,) + Bv.shape[1:]))
    check_gemm(np.ascontiguousarray(c[:, :, :N]), 0, tb, Ap, Bp, M, N, K, batch=batch)


def _raw_select(ta, tb, M, N, K, a_ptr, lda, b_ptr, ldb, c_ptr, kernel):
    return capi.raw_call("fdl_sgemm_ex_select", ta, tb, M, N, K, a_ptr, lda, 0, b_ptr, ldb, 0,
                         c_ptr, N, 0, 1, None, None, 0, kernel, stream())


@pytest.mark.parametrize("fam,bk", DMAS)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("K", [4, 20, 36, 52, 68, 100, 132, 196, 1000])
def test_dma_partial_last_k_tile(device, fam, bk, ta, tb, K):
    # K a multiple of 4 but not of the K-tile: the last tile's copies past K
    # are redirected and masked.  Non-finite values right at the end of K in
    # the other operand must not leak into the masked slots as 0 * inf.  The
    # K values give 1 to 5 K-tiles with a partial last one for each tile
    # depth (16, 32, 64), so the pipelined loop runs zero, one and several
    # steady-state tiles before its checked last tiles.
    M, N = 132, 200
    A, B = operands(_rng(K, ta, tb, fam), ta, tb, M, N, K, 1)
    say(f"dma partial K-tile fam={fam} ta={ta} tb={tb} K={K}")
    c = gpu_sgemm(ta, tb, A, B, M, N, K, kernel=fam)
    check_gemm(c, ta, tb, A, B, M, N, K)


@pytest.mark.parametrize("fam,bk", DMAS)
def test_dma_infinity_in_last_k_row(device, fam, bk):
    # B's last k row holds +inf in column 0: C[:, 0] must be +/-inf or nan
    # exactly where A[:, K-1] makes it so, and every other column finite.
    M, N, K = 64, 64, 36
    g = _rng(21, fam)
    A = np.abs(g.standard_normal((1, M, K))).astype(np.float32) + 0.5
    B = g.standard_normal((1, K, N)).astype(np.float32)
    B[0, K - 1, 0] = np.inf
    say(f"dma inf in last k row fam={fam}")
    c = gpu_sgemm(0, 0, A, B, M, N, K, kernel=fam)[0]
    assert np.all(np.isposinf(c[:, 0]))
    assert np.all(np.isfinite(c[:, 1:]))


def test_dma_refuses_unsupported_problems(device):
    import torch

    buf = torch.zeros(1 << 20, device="cuda")
    p = buf.data_ptr()
    big = torch.zeros(4 * ((1 << 22) + 4) + 64, device="cuda")
    pb = big.data_ptr()
    say("dma refusals")
    for fam, _ in DMAS16:
        # K not a multiple of 4
        assert _raw_select(0, 0, 64, 64, 22, p, 24, p, 64, p, fam) == -2
        assert "direct-to-LDS" in capi.last_error()
        # A misaligned by one float
        assert _raw_select(0, 0, 64, 64, 32, p + 4, 32, p, 64, p, fam) == -2
        # ld not a multiple of 4
        assert _raw_select(0, 0, 64, 64, 32, p, 33, p, 64, p, fam) == -2
        # N (B's contiguous extent) not a multiple of 4
        assert _raw_select(0, 0, 64, 66, 32, p, 32, p, 66, p, fam) == -2
        # leading dimension past 2^22 (the copies' 32-bit lane offsets); the
        # buffer covers what B's rows would span, so even a launch stays inside
        assert _raw_select(0, 0, 64, 64, 4, pb, 4, pb, (1 << 22) + 4, p, fam) == -2
        assert "2^22" in capi.last_error()
    for fam in (capi.KERNEL_DMA64U, capi.KERNEL_DMA128W8U, capi.KERNEL_DMA96X32U):
        # leading dimension past 2^24
        assert _raw_select(0, 0, 64, 64, 32, p, (1 << 24) + 1, p, 64, p, fam) == -2
        assert "4-byte" in capi.last_error()
        # A not even 4-byte aligned
        assert _raw_select(0, 0, 64, 64, 32, p + 2, 32, p, 64, p, fam) == -2
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K,fam", [(4096, 4096, 64, capi.KERNEL_DMA256),
                                        (2048, 2048, 64, capi.KERNEL_DMA128W8)])
def test_auto_choice_and_misaligned_fallback(device, M, N, K, fam):
    import torch

    assert capi.kernel_choice(0, 0, M, N, K) == fam
    g = _rng(17, M)
    A, B = operands(g, 0, 0, M, N, K, 1)
    # Operands placed one float past a 16-byte boundary: the automatic choice
    # must fall back to the register-staged kernel with the same tile and
    # still be right.
    dA = torch.zeros(M * K + 4, device="cuda")
    dB = torch.zeros(K * N + 4, device="cuda")
    dA[1:1 + M * K] = dev(A.reshape(-1))
    dB[1:1 + K * N] = dev(B.reshape(-1))
    dC = torch.full((M, N), float("nan"), device="cuda")
    say(f"auto {M}x{N}x{K} misaligned operands")
    capi.sgemm_ex(0, 0, M, N, K, dA.data_ptr() + 4, K, 0, dB.data_ptr() + 4, N, 0,
                  dC.data_ptr(), N, 0, 1, None, None, 0, stream())
    check_gemm(host(dC)[None], 0, 0, A, B, M, N, K)
    say(f"auto {M}x{N}x{K} aligned operands ({capi.KERNEL_NAMES[fam]})")
    dC.fill_(float("nan"))
    capi.sgemm_ex(0, 0, M, N, K, dA.data_ptr(), K, 0, dB.data_ptr(), N, 0,
                  dC.data_ptr(), N, 0, 1, None, None, 0, stream())
    # dA/dB hold the operands shifted by one element here, so recompute the
    # reference from what the aligned pointers see.
    A2 = host(dA)[:M * K].reshape(1, M, K)
    B2 = host(dB)[:K * N].reshape(1, K, N)
    check_gemm(host(dC)[None], 0, 0, A2, B2, M, N, K)
