"""Seeded random sweep of the automatic GEMM dispatch (fdl_sgemm_ex).

Each case draws the layouts, sizes (1 to about 2500, log-uniform), batch,
epilogue, padded leading dimensions, extra batch-stride slack and a pointer
offset of 0-3 floats (which sends 16-byte-copy choices to their 4-byte
twins), so the kernel families and their fallbacks are reached in
combinations the structured tests do not enumerate.  Every element must be
within the fp64 bound c0*(sqrt(K)+2)*eps*(|A||B|+|bias|) (oracle.gemm_tolerance),
computed in fp64 on the device, and every element of C outside the problem
(padding columns) must be left untouched.
"""
import numpy as np
import pytest

import fast_dl_amd.capi as capi
import oracle
from tests.gpu_helpers import say, stream

pytestmark = pytest.mark.gpu

N_CASES = 240


def _draw(g):
    ta, tb = int(g.integers(0, 2)), int(g.integers(0, 2))
    while True:
        M, N, K = (int(np.exp(g.uniform(0, np.log(2500)))) for _ in range(3))
        batch = int(g.choice([1, 1, 1, 2, 3]))
        if M * N * K * batch <= 2.5e9:
            break
    epi = int(g.integers(0, 5))
    pads = [int(g.choice([0, 0, 1, 3, 16])) for _ in range(3)]
    slack = [int(g.choice([0, 0, 4, 7])) for _ in range(3)]
    offs = [int(g.choice([0, 0, 0, 1, 2, 3])) for _ in range(2)]
    return ta, tb, M, N, K, batch, epi, pads, slack, offs


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_gemm_case(device, case):
    import torch

    g = np.random.default_rng(1000 + case)
    ta, tb, M, N, K, batch, epi, pads, slack, offs = _draw(g)
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    lda, ldb, ldc = a_cols + pads[0], b_cols + pads[1], N + pads[2]
    sA, sB, sC = a_rows * lda + slack[0], b_rows * ldb + slack[1], M * ldc + slack[2]
    say(f"random gemm case {case}: ta={ta} tb={tb} M={M} N={N} K={K} batch={batch} epi={epi} "
        f"ld=({lda},{ldb},{ldc}) slack={slack} offsets={offs}")
    gen = torch.Generator(device="cuda").manual_seed(case)
    # operands in flat buffers: element (b, r, c) at off + b*stride + r*ld + c
    bufA = torch.randn(offs[0] + batch * sA + 4, generator=gen, device="cuda")
    bufB = torch.randn(offs[1] + batch * sB + 4, generator=gen, device="cuda")
    bufC = torch.full((batch * sC + 4,), float("nan"), device="cuda")
    bias = torch.randn(N, generator=gen, device="cuda") * 0.5 if epi in (1, 2) else None
    auxbuf = torch.randn(batch * sC + 4, generator=gen, device="cuda") if epi == 4 else None
    capi.sgemm_ex(ta, tb, M, N, K, bufA.data_ptr() + 4 * offs[0], lda, sA,
                  bufB.data_ptr() + 4 * offs[1], ldb, sB, bufC.data_ptr(), ldc, sC, batch,
                  bias.data_ptr() if bias is not None else None,
                  auxbuf.data_ptr() if auxbuf is not None else None, epi, stream())

    def view(buf, off, stride, rows, ld, cols):
        return torch.as_strided(buf, (batch, rows, cols), (stride, ld, 1), off)

    A = view(bufA, offs[0], sA, a_rows, lda, a_cols).double()
    B = view(bufB, offs[1], sB, b_rows, ldb, b_cols).double()
    opA = A.transpose(1, 2) if ta else A
    opB = B.transpose(1, 2) if tb else B
    c64 = torch.bmm(opA.contiguous(), opB.contiguous())
    s64 = torch.bmm(opA.abs().contiguous(), opB.abs().contiguous())
    if bias is not None:
        c64 = c64 + bias.double()
        s64 = s64 + bias.double().abs()
    if epi in (2, 3):
        c64 = torch.clamp_min(c64, 0.0)
    if epi == 4:
        aux = view(auxbuf, 0, sC, M, ldc, N)
        c64 = torch.where(aux > 0, c64, torch.zeros_like(c64))
    got = view(bufC, 0, sC, M, ldc, N).double()
    # oracle.gemm_tolerance is linear in |A||B|: take its factor once, apply it on the device
    factor = float(oracle.gemm_tolerance(np.array([1.0]), K)[0])
    tol = s64 * factor + 1e-30
    err = (got - c64).abs()
    assert bool(torch.isfinite(got).all()), "unwritten or non-finite output"
    worst = float((err / tol).max()) if err.numel() else 0.0
    assert bool((err <= tol).all()), f"elementwise bound exceeded: max err/tol = {worst:.3f}"
    # padding columns and batch slack stay NaN (nothing written outside C)
    written = torch.zeros(batch * sC + 4, dtype=torch.bool, device="cuda")
    view(written, 0, sC, M, ldc, N).fill_(True)
    assert bool(torch.isnan(bufC[~written]).all()), "a store landed outside the problem"
