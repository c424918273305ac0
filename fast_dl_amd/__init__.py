"""fast_dl_amd -- MI355X (gfx950) fp32 GEMM path for fast_dl.

The product is the native library ``libfastdl_gemm.so`` (HIP kernels behind
the C-ABI in ``include/fastdl_gemm.h``) and the C++ ``dl::`` API built on it
(``libfastdl.so``).  This Python package only loads the C-ABI with ctypes so that
tests and ``bench.py`` can drive it with device buffers owned by PyTorch.
There is no Python or CPU fallback: if the library is missing, importing
:mod:`fast_dl_amd.capi` raises.
"""

from .capi import (  # noqa: F401
    EPILOGUE_BIAS,
    EPILOGUE_BIAS_RELU,
    EPILOGUE_NONE,
    EPILOGUE_RELU,
    EPILOGUE_RELU_GRAD,
    KERNEL_AUTO,
    KERNEL_DMA64,
    KERNEL_DMA128W8,
    KERNEL_DMA128W8U,
    KERNEL_DMA64U,
    KERNEL_DMA128,
    KERNEL_DMA256,
    KERNEL_SKINNY,
    KERNEL_SPLITK16,
    KERNEL_SPLITK32,
    KERNEL_TILED64,
    KERNEL_TILED128,
    KERNEL_TILED128W8,
    KERNEL_TILED256,
    KERNEL_TILED256X128,
    OP_N,
    OP_T,
    FdlError,
    library_path,
    load_library,
)
