"""CPU-side checks of the C-ABI library: it loads, exports every symbol the
public header declares, and rejects invalid arguments before touching a GPU
(validation never calls into the HIP runtime)."""
import ctypes
import glob
import os
import re

import numpy as np

import fast_dl_amd.capi as capi
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fdl_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_header_symbols():
    lib = capi.load_library()
    assert [os.path.basename(h) for h in HEADERS] == ["fastdl_data.h", "fastdl_gemm.h"]
    names = [n for h in HEADERS for n in declared_functions(h)]
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/*.h but not exported"
        assert name in capi.SIGNATURES, f"{name} missing from the ctypes binding"
    assert "gfx950" in capi.version()


def test_status_strings():
    lib = capi.load_library()
    assert lib.fdl_status_string(0) == b"FDL_SUCCESS"
    assert lib.fdl_status_string(-1) == b"FDL_ERROR_INVALID_VALUE"


def _sgemm_status(**kw):
    args = dict(ta=0, tb=0, M=4, N=4, K=4, A=1 << 20, lda=4, sA=0, B=1 << 20, ldb=4, sB=0,
                C=1 << 20, ldc=4, sC=0, batch=1, bias=None, aux=None, epi=0, stream=None)
    args.update(kw)
    return capi.raw_call("fdl_sgemm_ex", *args.values())


def test_sgemm_argument_validation():
    bad = [
        dict(ta=2), dict(tb=-1), dict(M=-1), dict(K=1 << 31), dict(batch=-1), dict(epi=7),
        dict(lda=3), dict(ldb=3), dict(ldc=3), dict(ta=1, lda=3), dict(tb=1, ldb=3),
        dict(sA=-4), dict(batch=2, sC=4), dict(C=None), dict(A=None), dict(B=None),
        dict(epi=1), dict(epi=2), dict(epi=4),
    ]
    for kw in bad:
        assert _sgemm_status(**kw) == -1, kw
        assert capi.last_error().startswith("sgemm:")


def test_noop_sizes_need_no_gpu():
    # M == 0, N == 0 or batch == 0: valid and nothing is launched
    assert _sgemm_status(M=0, A=None, B=None, C=None) == 0
    assert _sgemm_status(N=0, lda=4, ldb=1, ldc=1, A=None, B=None, C=None) == 0
    assert _sgemm_status(batch=0, A=None, B=None, C=None) == 0


def test_other_entry_points_validate():
    assert capi.raw_call("fdl_gemm", None, None, None, -1, 2, 2) == -1
    assert capi.raw_call("fdl_relu", None, None, 5, None) == -1
    assert capi.raw_call("fdl_relu", None, None, 0, None) == 0
    assert capi.raw_call("fdl_colsum", None, None, 3, 3, None) == -1
    assert capi.raw_call("fdl_softmax", 1, 1, 0, 3, None) == -1
    assert capi.raw_call("fdl_softmax_xent", 1, 1, 1, 1, 4, 0, None) == -1
    assert "class count" in capi.last_error()
    assert capi.raw_call("fdl_sgd_update", None, None, 0.1, -1, None) == -1
    assert capi.raw_call("fdl_sgemm_ex_select", 0, 1, 16, 16, 16, 1, 16, 0, 1, 16, 0, 1, 16, 0,
                         1, None, None, 0, 3, None) == -2  # skinny with B transposed
    assert capi.raw_call("fdl_sgemm_ex_select", 0, 0, 16, 16, 16, 1, 16, 0, 1, 16, 0, 1, 16, 0,
                         1, None, None, 0, 16, None) == -1
    assert capi.raw_call("fdl_sgemm_ex_select", 0, 0, 16, 16, 22, 1 << 20, 24, 0, 1 << 20, 16, 0,
                         1 << 20, 16, 0, 1, None, None, 0, capi.KERNEL_DMA256, None) == -2
    assert capi.raw_call("fdl_mlp2_train_step", *([None] * 2), 0, 1, 1, 1, *([None] * 4), 0.1,
                         *([None] * 11)) == -1
    # a graph of no steps is refused before any capture
    handle = ctypes.c_void_p()
    assert capi.raw_call("fdl_mlp2_graph_create_steps", ctypes.byref(handle), 0, *([None] * 2),
                         256, 784, 256, 10, *([None] * 4), 0.1, *([None] * 11)) == -1
    assert "steps" in capi.last_error() and handle.value is None


def test_kernel_choice():
    assert capi.kernel_choice(0, 0, 4096, 4096, 4096) == capi.KERNEL_DMA256
    # every layout: the four-wave 256x256 tile (TT 4096^3: 899 us, against 970
    # us for the 64x64 tile)
    assert capi.kernel_choice(1, 1, 4096, 4096, 4096) == capi.KERNEL_DMA256
    # K not a multiple of 4, or B's contiguous extent not a multiple of 4:
    # the 4-byte-copy direct-to-LDS tiles
    assert capi.kernel_choice(0, 0, 4096, 4096, 4098) == capi.KERNEL_DMA128W8U
    assert capi.kernel_choice(0, 0, 4096, 4094, 4096) == capi.KERNEL_DMA128W8U
    # a partial last K-tile is fine for the direct-to-LDS kernels
    assert capi.kernel_choice(0, 0, 4096, 4096, 4100) == capi.KERNEL_DMA256
    # mid-size cubes: the 64x64 direct-to-LDS tile where K % 4 == 0
    assert capi.kernel_choice(0, 0, 1024, 1024, 1024) == capi.KERNEL_DMA64
    assert capi.kernel_choice(0, 0, 1000, 1000, 1000) == capi.KERNEL_DMA64
    assert capi.kernel_choice(0, 0, 1023, 1023, 1023) == capi.KERNEL_DMA64U
    # 777^3: 169 tiles of 64x64 leave 87 CUs idle; 225 tiles of 96x32 do not
    assert capi.kernel_choice(0, 0, 777, 777, 777) == capi.KERNEL_DMA96X32U
    assert capi.kernel_choice(0, 0, 700, 900, 800) == capi.KERNEL_DMA96X32U
    # short K: a full GPU of 64x64 tiles takes the four-stage 64x64x16 tile
    # (the C4 batch), a tile count just past one round stays on split-K
    assert capi.kernel_choice(0, 0, 128, 128, 64, 64) == capi.KERNEL_DMA64S
    assert capi.kernel_choice(0, 1, 128, 128, 64, 64) == capi.KERNEL_DMA64S
    assert capi.kernel_choice(0, 0, 1024, 1024, 128) == capi.KERNEL_DMA64S
    assert capi.kernel_choice(0, 0, 1024, 1024, 256) == capi.KERNEL_DMA64
    assert capi.kernel_choice(0, 1, 1000, 1100, 96) == capi.KERNEL_SPLITK32
    assert capi.kernel_choice(0, 0, 1024, 1024, 32) == capi.KERNEL_SPLITK32
    # about one 128x128 tile per CU: the 128x128 tile of FDL_KERNEL_DMA128W8
    # (its four-wave hand-scheduled form on NN); three per CU as well on NN
    # (4000x3000x2048: 361 us against 373 us for the two-blocks-per-CU tile)
    assert capi.kernel_choice(0, 0, 2048, 2048, 2048) == capi.KERNEL_DMA128W8
    assert capi.kernel_choice(0, 0, 4000, 3000, 2048) == capi.KERNEL_DMA128W8
    # K not a multiple of 4 rules the direct-to-LDS tiles out
    assert capi.kernel_choice(0, 0, 2048, 2048, 2050) not in (capi.KERNEL_DMA128,
                                                              capi.KERNEL_DMA256,
                                                              capi.KERNEL_DMA64,
                                                              capi.KERNEL_DMA128W8)
    assert capi.kernel_choice(0, 0, 8, 4096, 4096) == capi.KERNEL_SKINNY
    assert capi.kernel_choice(0, 1, 8, 4096, 4096) != capi.KERNEL_SKINNY
    assert capi.kernel_choice(0, 0, 256, 128, 784) == capi.KERNEL_SPLITK16


def test_golden_fixtures_reproduced_by_oracle():
    import hashlib

    gold = np.load(os.path.join(ROOT, "tests", "golden", "config1_gemm.npz"))
    g = np.random.default_rng(1)
    A = g.random((1, 256, 784)).astype(np.float32)
    B = (g.standard_normal((1, 784, 128)) * np.sqrt(2.0 / 784)).astype(np.float32)
    assert hashlib.sha256(A.tobytes()).digest() == gold["sha_A"].tobytes()
    assert hashlib.sha256(B.tobytes()).digest() == gold["sha_B"].tobytes()
    assert np.array_equal(oracle.gemm_cpu(A[0], B[0]), gold["C32"])
    c64 = A[0].astype(np.float64) @ B[0].astype(np.float64)
    assert np.allclose(gold["C64"], c64, rtol=1e-12, atol=1e-12)

    m = np.load(os.path.join(ROOT, "tests", "golden", "mlp2_small_step.npz"))
    out = oracle.mlp2_train_step(m["X"], m["labels"], m["W1"], m["b1"], m["W2"], m["b2"],
                                 float(m["lr"]))
    for k in ("W1", "b1", "W2", "b2", "dX", "loss"):
        assert np.array_equal(out[k], m[f"out_{k}"]), k


def _gather_status(**kw):
    args = dict(images=1 << 20, labels=1 << 20, count=10, row_bytes=784, index=None, batch=4,
                divisor=255.0, x=1 << 20, y=1 << 20, stream=None)
    args.update(kw)
    return capi.raw_call("fdl_idx_gather", *args.values())


def test_idx_gather_argument_validation():
    bad = [
        dict(count=-1), dict(row_bytes=-1), dict(batch=-1), dict(divisor=0.0),
        dict(divisor=float("inf")), dict(divisor=float("nan")), dict(x=None, y=None),
        dict(images=None), dict(labels=None), dict(batch=11),
        dict(row_bytes=1 << 40, count=1 << 30),
    ]
    for kw in bad:
        assert _gather_status(**kw) == -1, kw
        assert capi.last_error().startswith("idx_gather:")
    # no-ops and inputs that may be null: nothing is launched
    assert _gather_status(batch=0, images=None, labels=None, x=None, y=None) == 0


def test_workspace_size():
    # the skinny family's K split: 256-column bands x K slices x M rows rounded
    # up to 1, 2, 4 or 8, in floats; about 416 blocks at M <= 2, 512 above
    assert capi.workspace_size(0, 0, 1, 4096, 4096) == 16 * 26 * 1 * 256 * 4
    assert capi.workspace_size(0, 0, 8, 4096, 4096) == 16 * 32 * 8 * 256 * 4
    assert capi.workspace_size(1, 0, 3, 4096, 4096) == 16 * 32 * 4 * 256 * 4
    assert capi.workspace_size(0, 0, 1, 1024, 16384) == 4 * 64 * 256 * 4
    assert capi.workspace_size(0, 0, 8, 16384, 1024) > 0     # 64 MB of B
    assert capi.workspace_size(0, 0, 4, 4096, 1024) == 0     # 16 MB, short K: single pass
    assert capi.workspace_size(0, 1, 1, 4096, 4096) == 0     # B transposed
    assert capi.workspace_size(0, 0, 1, 4096, 4096, 2) == 0  # batched
    assert capi.workspace_size(0, 0, 9, 4096, 4096) == 0     # not skinny
    assert capi.workspace_size(0, 0, 1, 4098, 4096) == 0     # N % 4 != 0
    assert capi.workspace_size(0, 0, 1, 4096, 4096, 0) == 0


def test_workspace_validation():
    args = [0, 0, 1, 4096, 4096, 1 << 20, 4096, 0, 1 << 20, 4096, 0, 1 << 20, 4096, 0, 1,
            None, None, 0]
    assert capi.raw_call("fdl_sgemm_ex_ws", *args, (1 << 20) + 4, 1 << 20, None) == -1
    assert "16-byte aligned" in capi.last_error()
