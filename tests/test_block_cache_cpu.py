"""The tensor block cache's bookkeeping on the host (no GPU).

tests/cpp/host/block_cache_test.cpp drives fast_dl_amd/csrc/dl/tensor/block_cache.hpp
with a fake device backend: freed blocks return to the stream they were
allocated on, blocks used on other streams wait for markers, retired streams
hand their blocks to a shared pool, and an out-of-memory allocation frees the
cache and retries once.  Built with the address and undefined-behaviour
sanitizers (host code only).
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_block_cache_bookkeeping(tmp_path):
    exe = tmp_path / "block_cache_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror",
                    "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-I", os.path.join(ROOT, "fast_dl_amd", "csrc", "dl", "tensor"),
                    os.path.join(ROOT, "tests", "cpp", "host", "block_cache_test.cpp"),
                    "-o", str(exe)], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "not passed" not in proc.stdout
    assert "block_cache_test : passed" in proc.stdout


def test_stream_use_list_threads(tmp_path):
    """TensorImpl's list of the streams a tensor is used on, recorded from several
    threads at once (a shared weight read by threads on their own streams), under the
    thread sanitizer."""
    exe = tmp_path / "stream_use_list_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror",
                    "-fsanitize=thread", "-pthread", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "host", "stream_use_list_test.cpp"),
                    "-o", str(exe)], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "WARNING: ThreadSanitizer" not in proc.stderr, proc.stderr
    assert "stream_use_list_test : passed" in proc.stdout
