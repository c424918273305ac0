"""fast_dl_amd -- MI355X (gfx950) fp32 GEMM path for fast_dl.

The product is the native library ``libfastdl_gemm.so`` (HIP kernels behind
the C-ABI in ``include/fastdl_gemm.h``) and the C++ ``dl::`` API built on it
(``libfastdl.so``).  This Python package only loads the C-ABI with ctypes so that
tests and ``bench.py`` can drive it with device buffers owned by PyTorch.
There is no Python or CPU fallback: if the library is missing,
:func:`fast_dl_amd.capi.load_library` (which every call goes through) raises.
"""
