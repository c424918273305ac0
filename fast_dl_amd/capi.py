"""ctypes binding of ``include/fastdl_gemm.h``.

Every function takes raw device addresses (ints, e.g. ``tensor.data_ptr()``)
and a raw ``hipStream_t`` (int, e.g. ``torch.cuda.current_stream().cuda_stream``,
0 for the null stream).  Non-zero statuses raise :class:`FdlError` carrying
the library's own message.
"""
from __future__ import annotations

import ctypes
import os

OP_N, OP_T = 0, 1
EPILOGUE_NONE, EPILOGUE_BIAS, EPILOGUE_BIAS_RELU, EPILOGUE_RELU, EPILOGUE_RELU_GRAD = range(5)
KERNEL_AUTO, KERNEL_TILED128, KERNEL_TILED64, KERNEL_SPLITK32, KERNEL_SKINNY = -1, 0, 1, 2, 3
KERNEL_TILED256, KERNEL_TILED256X128, KERNEL_TILED128W8, KERNEL_SPLITK16 = 4, 5, 6, 7
KERNEL_DMA256, KERNEL_DMA128, KERNEL_DMA64, KERNEL_DMA128W8 = 8, 9, 10, 11
KERNEL_DMA64U, KERNEL_DMA128W8U, KERNEL_DMA64S, KERNEL_DMA96X32U = 12, 13, 14, 15
KERNEL_NAMES = {KERNEL_TILED128: "tiled128", KERNEL_TILED64: "tiled64",
                KERNEL_SPLITK32: "splitk32", KERNEL_SKINNY: "skinny", KERNEL_TILED256: "tiled256",
                KERNEL_TILED256X128: "tiled256x128", KERNEL_TILED128W8: "tiled128w8",
                KERNEL_SPLITK16: "splitk16", KERNEL_DMA256: "dma256", KERNEL_DMA128: "dma128",
                KERNEL_DMA64: "dma64", KERNEL_DMA128W8: "dma128w8", KERNEL_DMA64U: "dma64u",
                KERNEL_DMA128W8U: "dma128w8u", KERNEL_DMA64S: "dma64s",
                KERNEL_DMA96X32U: "dma96x32u"}

_PKG = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_flt = ctypes.c_float

# name -> (restype, argtypes); mirrors include/fastdl_gemm.h and include/fastdl_data.h.
SIGNATURES = {
    "fdl_sgemm_ex": (_int, [_int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                            _vp, _i64, _i64, _i64, _vp, _vp, _int, _vp]),
    "fdl_sgemm_ex_select": (_int, [_int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                   _i64, _vp, _i64, _i64, _i64, _vp, _vp, _int, _int, _vp]),
    "fdl_sgemm_kernel_choice": (_int, [_int, _int, _i64, _i64, _i64, _i64]),
    "fdl_sgemm_workspace_size": (ctypes.c_size_t, [_int, _int, _i64, _i64, _i64, _i64]),
    "fdl_sgemm_ex_noalloc": (_int, [_int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                    _i64, _vp, _i64, _i64, _i64, _vp, _vp, _int, _vp]),
    "fdl_sgemm_ex_ws": (_int, [_int, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                               _vp, _i64, _i64, _i64, _vp, _vp, _int, _vp, ctypes.c_size_t,
                               _vp]),
    "fdl_gemm": (_int, [_vp, _vp, _vp, _int, _int, _int]),
    "fdl_add_row_bias": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "fdl_relu": (_int, [_vp, _vp, _i64, _vp]),
    "fdl_relu_backward": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "fdl_colsum": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "fdl_softmax": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "fdl_softmax_xent": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fdl_sgd_update": (_int, [_vp, _vp, _flt, _i64, _vp]),
    "fdl_mlp2_train_step": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _flt,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "fdl_mlp2_graph_create": (_int, [ctypes.POINTER(_vp), _vp, _vp, _i64, _i64, _i64, _i64,
                                     _vp, _vp, _vp, _vp, _flt, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _vp, _vp]),
    "fdl_mlp2_graph_create_steps": (_int, [ctypes.POINTER(_vp), _int, _vp, _vp, _i64, _i64,
                                           _i64, _i64, _vp, _vp, _vp, _vp, _flt, _vp, _vp,
                                           _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "fdl_mlp2_graph_launch": (_int, [_vp, _vp]),
    "fdl_mlp2_graph_destroy": (_int, [_vp]),
    "fdl_zero_fill": (_int, [_vp, _i64, _vp]),
    "fdl_fill_uniform": (_int, [_vp, _i64, _flt, _flt, ctypes.c_uint64, _vp]),
    "fdl_fill_normal": (_int, [_vp, _i64, _flt, _flt, ctypes.c_uint64, _vp]),
    "fdl_idx_gather": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _flt, _vp, _vp, _vp]),
    "fdl_last_error": (ctypes.c_char_p, []),
    "fdl_status_string": (ctypes.c_char_p, [_int]),
    "fdl_version": (ctypes.c_char_p, []),
}


class FdlError(RuntimeError):
    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


def library_path() -> str:
    return os.path.join(_PKG, "libfastdl_gemm.so")


def load_library() -> ctypes.CDLL:
    """Load ``libfastdl_gemm.so``; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _checked(name: str):
    def call(*args):
        lib = load_library()
        status = getattr(lib, name)(*args)
        if status != 0:
            raise FdlError(name, status, lib.fdl_last_error().decode())
        return status
    call.__name__ = name
    return call


sgemm_ex = _checked("fdl_sgemm_ex")
sgemm_ex_select = _checked("fdl_sgemm_ex_select")
sgemm_ex_ws = _checked("fdl_sgemm_ex_ws")
sgemm_ex_noalloc = _checked("fdl_sgemm_ex_noalloc")
gemm = _checked("fdl_gemm")
add_row_bias = _checked("fdl_add_row_bias")
relu = _checked("fdl_relu")
relu_backward = _checked("fdl_relu_backward")
colsum = _checked("fdl_colsum")
softmax = _checked("fdl_softmax")
softmax_xent = _checked("fdl_softmax_xent")
sgd_update = _checked("fdl_sgd_update")
mlp2_train_step = _checked("fdl_mlp2_train_step")
fill_uniform = _checked("fdl_fill_uniform")
mlp2_graph_launch = _checked("fdl_mlp2_graph_launch")
mlp2_graph_destroy = _checked("fdl_mlp2_graph_destroy")


fill_normal = _checked("fdl_fill_normal")
idx_gather = _checked("fdl_idx_gather")


def mlp2_graph_create(*args) -> int:
    """Capture fdl_mlp2_train_step(*args) into a graph; returns the handle (an int)."""
    handle = ctypes.c_void_p()
    lib = load_library()
    status = lib.fdl_mlp2_graph_create(ctypes.byref(handle), *args)
    if status != 0:
        raise FdlError("fdl_mlp2_graph_create", status, lib.fdl_last_error().decode())
    return handle.value


def mlp2_graph_create_steps(steps: int, *args) -> int:
    """Capture `steps` consecutive fdl_mlp2_train_step(*args) calls into one graph."""
    handle = ctypes.c_void_p()
    lib = load_library()
    status = lib.fdl_mlp2_graph_create_steps(ctypes.byref(handle), steps, *args)
    if status != 0:
        raise FdlError("fdl_mlp2_graph_create_steps", status, lib.fdl_last_error().decode())
    return handle.value


def kernel_choice(transA: int, transB: int, M: int, N: int, K: int, batch: int = 1) -> int:
    return load_library().fdl_sgemm_kernel_choice(transA, transB, M, N, K, batch)


def workspace_size(transA: int, transB: int, M: int, N: int, K: int, batch: int = 1) -> int:
    """Bytes of workspace fdl_sgemm_ex_ws can use for this problem (0: none)."""
    return load_library().fdl_sgemm_workspace_size(transA, transB, M, N, K, batch)


def version() -> str:
    return load_library().fdl_version().decode()


def raw_call(name: str, *args) -> int:
    """Call an entry point and return its status without raising (for error-path tests)."""
    return getattr(load_library(), name)(*args)


def last_error() -> str:
    return load_library().fdl_last_error().decode()
