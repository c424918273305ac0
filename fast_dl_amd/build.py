"""Build recipe for the native libraries, driven by ``__graft_entry__.build()``.

Compiles, in-tree, with hipcc for gfx950 only:

* ``fast_dl_amd/libfastdl_gemm.so`` -- HIP kernels + the C-ABI declared in
  ``include/fastdl_gemm.h`` and ``include/fastdl_data.h``;
* ``fast_dl_amd/libfastdl.so`` -- the C++ ``dl::`` tensor/ops/nn API
  (``include/dl``) hosted on the HIP runtime, linked against the former;
* the C++ API test programs under ``tests/cpp`` (``tests/cpp/bin``).

Every call rebuilds everything (the driver uses this as the "does it build"
check).  Object files go to ``fast_dl_amd/_build`` (git-ignored).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops keeps the compiler from emitting v_pk_{add,mul,fma}_f32.
# Kernel-argument preloading (gfx950): the first kernel arguments arrive in
# SGPRs at wave launch instead of through scalar loads from the argument
# buffer, which a kernel's first instructions otherwise wait for (the MLP
# step 17.00 -> 16.91 us, C1 4.32 -> 4.26 us back to back, alternated on one
# GPU).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]
COMMON_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-result",
                "-I", INCLUDE, "-I", CSRC]

GEMM_SOURCES = ["sgemm.hip", "mlp_kernels.hip", "data_kernels.hip", "capi.hip"]
DL_SOURCES_DIR = os.path.join(CSRC, "dl")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        # hipcc's host pass does not know the device-only feature flag.
        if "packed-fp32-ops" not in line and "not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
# Host-only C++ (the dl:: API) is plain C++17 against the HIP runtime API.
HOST_CXX = os.environ.get("CXX_HOST", "g++")
HOST_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
              "-I", INCLUDE, "-I", os.path.join(ROCM, "include")]


def _compile(src: str, obj: str, device: bool) -> str:
    if device:
        cmd = [HIPCC, *COMMON_FLAGS, *DEVICE_FLAGS, "-c", src, "-o", obj]
    else:
        cmd = [HOST_CXX, *HOST_FLAGS, "-c", src, "-o", obj]
    _run(cmd)
    return obj


def _jobs() -> int:
    return max(1, min(16, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))


def build_gemm_library() -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in GEMM_SOURCES]
    objs = [os.path.join(BUILD, os.path.basename(s) + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(_jobs()) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], True), zip(srcs, objs)))
    out = os.path.join(PKG, "libfastdl_gemm.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def build_dl_library() -> str | None:
    srcs = sorted(glob.glob(os.path.join(DL_SOURCES_DIR, "**", "*.cpp"), recursive=True))
    if not srcs:
        return None
    os.makedirs(BUILD, exist_ok=True)
    objs = [os.path.join(BUILD, "dl_" + os.path.relpath(s, DL_SOURCES_DIR).replace(os.sep, "_") + ".o")
            for s in srcs]
    # Host-only C++ on the HIP runtime API (no kernels in these files).
    with cf.ThreadPoolExecutor(_jobs()) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], False), zip(srcs, objs)))
    out = os.path.join(PKG, "libfastdl.so")
    tmp = out + ".tmp"
    _run([HOST_CXX, "-shared", "-fPIC", "-o", tmp, *objs,
          "-L", PKG, "-lfastdl_gemm", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, out)
    return out


def build_cpp_tests() -> list[str]:
    test_dir = os.path.join(ROOT, "tests", "cpp")
    srcs = sorted(glob.glob(os.path.join(test_dir, "*.cpp")))
    if not srcs:
        return []
    bindir = os.path.join(test_dir, "bin")
    os.makedirs(bindir, exist_ok=True)

    def one(src: str) -> str:
        exe = os.path.join(bindir, os.path.splitext(os.path.basename(src))[0])
        # The HIP runtime API too: a test may drive streams and graphs itself.
        _run([HOST_CXX, "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", INCLUDE,
              "-I", os.path.join(ROCM, "include"), src, "-o", exe,
              "-L", PKG, "-lfastdl", "-lfastdl_gemm",
              "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
              "-Wl,-rpath,$ORIGIN/../../../fast_dl_amd", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
        return exe

    with cf.ThreadPoolExecutor(_jobs()) as ex:
        return list(ex.map(one, srcs))


def build_all(verbose: bool = True) -> None:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    lib = build_gemm_library()
    if verbose:
        print(f"built {lib}")
    dl = build_dl_library()
    if dl and verbose:
        print(f"built {dl}")
    exes = build_cpp_tests() if dl else []
    if exes and verbose:
        print(f"built {len(exes)} C++ API test programs")


if __name__ == "__main__":
    build_all()
