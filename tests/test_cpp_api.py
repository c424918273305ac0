"""The C++ dl:: API: headers, exported symbols (CPU) and the C++ test programs (GPU).

The GPU part runs tests/cpp/bin/api_test (this build's own checks) and the
reference's own C++ test programs from /root/reference/tests, compiled
unchanged against this repository's include/dl and libfastdl.so by
`make -C oracle ref` (oracle/_ref/, built where the reference is mounted and
shipped prebuilt to the GPU box).  Each prints "<name> : passed".
"""
import glob
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "fast_dl_amd", "libfastdl.so")

PUBLIC_HEADERS = [
    "dl/dl.hpp", "dl/core/Device.hpp", "dl/core/DType.hpp", "dl/core/Shape.hpp",
    "dl/tensor/Tensor.hpp", "dl/tensor/TensorImpl.hpp", "dl/ops/Ops.hpp", "dl/ops/OpUtils.hpp",
    "dl/nn/Module.hpp", "dl/nn/Linear.hpp", "dl/nn/ReLU.hpp", "dl/nn/Sequential.hpp",
    "dl/kernels/kernels.hpp", "dl/optim/SGD.hpp", "dl/train/Mlp2.hpp", "dl/core/Stream.hpp",
    "dl/data/DataLoader.hpp", "dl/autograd/Node.hpp", "dl/train/Epoch.hpp",
]


@pytest.mark.parametrize("header", PUBLIC_HEADERS)
def test_public_headers_are_plain_cxx(header, tmp_path):
    # No HIP (or CUDA) headers needed to use the API, as in the reference.
    src = tmp_path / "h.cpp"
    src.write_text(f"#include <{header}>\nint main() {{ return 0; }}\n")
    subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", INCLUDE, str(src)], check=True)


REFERENCE_ALGO_NAMES = """
#include <dl/kernels/gemm.hpp>
#include <cstdio>
#include <cstring>
#include <initializer_list>

// The reference's own spellings: src/ops/Matmul.cpp:42 passes GemmAlgo::Cublas to
// gemm(), tests/benchmarks/gemm/gemm_benchmark.cu:87-99 runs each of the four.  Never
// called here (no GPU); it only has to compile and link.
void reference_calls(const float* a, const float* b, float* c, int m, int n, int k) {
    dl::kernels::gemm(a, b, c, m, n, k, dl::kernels::GemmAlgo::Cublas);
    for (auto algo : {dl::kernels::GemmAlgo::Naive, dl::kernels::GemmAlgo::Tiled,
                      dl::kernels::GemmAlgo::Register, dl::kernels::GemmAlgo::Cublas}) {
        dl::kernels::gemm(a, b, c, m, n, k, algo);
    }
}

int main() {
    // to_string as the reference's gemm.cu:183-195 spells it
    const struct { dl::kernels::GemmAlgo algo; const char* name; } names[] = {
        {dl::kernels::GemmAlgo::Naive, "naive"}, {dl::kernels::GemmAlgo::Tiled, "tiled"},
        {dl::kernels::GemmAlgo::Register, "register"}, {dl::kernels::GemmAlgo::Cublas, "cublas"}};
    for (const auto& e : names) {
        if (std::strcmp(dl::kernels::to_string(e.algo), e.name) != 0) {
            std::printf("to_string mismatch: %s\\n", e.name);
            return 1;
        }
    }
    std::printf("reference algo names ok\\n");
    return reference_calls == nullptr;
}
"""


def test_reference_gemm_algo_names_compile_and_print(tmp_path):
    """A caller written against the reference's GemmAlgo (Naive, Tiled, Register, Cublas)
    compiles and links unchanged, and to_string gives the reference's names."""
    assert os.path.exists(LIB), "libfastdl.so not built"
    src = tmp_path / "algo_names.cpp"
    src.write_text(REFERENCE_ALGO_NAMES)
    exe = tmp_path / "algo_names"
    pkg = os.path.dirname(LIB)
    subprocess.run(["g++", "-std=c++17", "-I", INCLUDE, str(src), "-o", str(exe), "-L", pkg,
                    "-lfastdl", "-lfastdl_gemm", f"-Wl,-rpath,{pkg}"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "reference algo names ok" in out.stdout


REFERENCE_ROOT = "/root/reference"


@pytest.mark.skipif(not os.path.isdir(REFERENCE_ROOT), reason="reference sources not mounted")
def test_every_gemm_algo_the_reference_names_compiles(tmp_path):
    """Every `GemmAlgo::X` spelled anywhere in the reference's sources (src/ops/Matmul.cpp:42,
    tests/benchmarks/gemm/gemm_benchmark.cu:87-99, ...) names an enumerator of this build's
    dl/kernels/gemm.hpp.  The files themselves include CUDA headers (cuda_runtime.h,
    dl/core/CudaUtils.hpp), so they are scanned as text, not compiled."""
    import re
    names = set()
    for path in glob.glob(os.path.join(REFERENCE_ROOT, "**", "*.*"), recursive=True):
        if os.path.splitext(path)[1] not in (".cpp", ".cu", ".hpp", ".cuh", ".h"):
            continue
        with open(path, errors="replace") as f:
            names.update(re.findall(r"GemmAlgo::(\w+)", f.read()))
    assert {"Naive", "Tiled", "Register", "Cublas"} <= names, sorted(names)
    src = tmp_path / "names.cpp"
    body = "\n".join(f"    (void)dl::kernels::to_string(dl::kernels::GemmAlgo::{n});"
                     for n in sorted(names))
    src.write_text(f"#include <dl/kernels/gemm.hpp>\nvoid f() {{\n{body}\n}}\n")
    subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", INCLUDE, str(src)], check=True)


def test_library_exports_api_symbols():
    assert os.path.exists(LIB), "libfastdl.so not built"
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    for sym in ["dl::ops::matmul(dl::Tensor const&, dl::Tensor const&)",
                "dl::ops::linear(dl::Tensor const&, dl::Tensor const&, dl::Tensor const&)",
                "dl::ops::relu(dl::Tensor const&)",
                "dl::ops::softmax(dl::Tensor const&)",
                "dl::ops::cross_entropy(dl::Tensor const&, dl::Tensor const&)",
                "dl::kernels::gemm(float const*, float const*, float*, int, int, int, "
                "dl::kernels::GemmAlgo)",
                "dl::kernels::add_row_bias(float*, float const*, int, int)",
                "dl::nn::Linear::forward(dl::Tensor const&)",
                "dl::Tensor::kaiming_uniform(dl::Shape, dl::DType, dl::Device, unsigned long)",
                "dl::ops::linear_backward(",
                "dl::current_stream()", "dl::StreamGuard::StreamGuard(void*)",
                "dl::Stream::Stream(dl::Device const&)",
                "dl::train::Mlp2::capture(dl::Tensor const&, dl::Tensor const&, float)",
                "dl::train::Mlp2::capture(dl::Tensor const&, dl::Tensor const&, float, int)",
                "dl::train::Mlp2::replay(bool)",
                "dl::data::DataLoader::DataLoader(std::__cxx11::basic_string<",
                "dl::data::DataLoader::gather(dl::Tensor const&, long, long, dl::Tensor&, "
                "dl::Tensor&)",
                "dl::data::DataLoader::getImagesMatrix(dl::Device const&)",
                "dl::Tensor::backward() const", "dl::Tensor::grad() const",
                "dl::train::train_epoch(",
                "dl::Tensor::set_requires_grad(bool)",
                "dl::optim::SGD::step(std::vector<dl::Tensor*, std::allocator<dl::Tensor*> > const&) const"]:
        assert sym in out, sym


def _programs():
    progs = sorted(glob.glob(os.path.join(ROOT, "tests", "cpp", "bin", "*")))
    progs += sorted(glob.glob(os.path.join(ROOT, "oracle", "_ref", "*")))
    return [p for p in progs if os.access(p, os.X_OK) and os.path.isfile(p)]


@pytest.mark.gpu
@pytest.mark.parametrize("prog", _programs(), ids=lambda p: os.path.relpath(p, ROOT))
def test_cpp_program(device, prog):
    print(f"running {prog}", flush=True)
    proc = subprocess.run([prog], capture_output=True, text=True, timeout=100)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "not passed" not in proc.stdout
    assert "passed" in proc.stdout
