"""The CMake build (CMakeLists.txt, LANGUAGES CXX HIP, gfx950): it configures,
builds the library, the harness and the oracle, registers the ctests,
installs a CMake package, and a downstream project finds it with
find_package(fa_mi355x) and links fa_mi355x::fa_mi355x. Host-only checks
(the ctests themselves need the GPU). The library exports the same C-ABI
symbols as the in-tree Python build."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"


def _defined_c_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.split() and line.split()[-1].startswith("fa_")}


@pytest.mark.skipif(not (shutil.which("cmake") and os.path.exists(CLANG)), reason="cmake or ROCm clang missing")
def test_cmake_build_install_and_consume(tmp_path, fa_lib):
    build, prefix, consumer = tmp_path / "build", tmp_path / "prefix", tmp_path / "consumer"

    def run(*cmd, cwd=None):
        res = subprocess.run(list(map(str, cmd)), cwd=cwd, capture_output=True, text=True)
        assert res.returncode == 0, (cmd, res.stdout[-3000:], res.stderr[-3000:])
        return res.stdout

    run("cmake", "-S", REPO, "-B", build, f"-DCMAKE_HIP_COMPILER={CLANG}")
    run("cmake", "--build", build, "-j8")
    tests = run("ctest", "--test-dir", build, "-N")
    for name in ("flash_attention_accuracy", "flash_attention_bench_quick", "v0_profile_correctness"):
        assert name in tests
    assert _defined_c_symbols(build / "libfa_mi355x.so") == _defined_c_symbols(fa_lib.LIB_PATH)
    run("cmake", "--install", build, "--prefix", prefix)

    consumer.mkdir()
    (consumer / "CMakeLists.txt").write_text(
        "cmake_minimum_required(VERSION 3.21)\nproject(consumer LANGUAGES CXX)\n"
        "find_package(fa_mi355x REQUIRED CONFIG)\nadd_executable(consumer main.cpp)\n"
        "target_link_libraries(consumer PRIVATE fa_mi355x::fa_mi355x)\n")
    (consumer / "main.cpp").write_text(
        '#include "flash_attention.h"\n#include <cstdio>\n'
        "int main() {\n  using namespace cuda_op_lab::flash_attention;\n"
        '  std::printf("%.0f %d\\n", attention_flops(AttentionShape{2, 8, 2048, 128}, false),\n'
        "              (int)tensorcore_v3_supported(128));\n  return 0;\n}\n")
    run("cmake", "-S", consumer, "-B", consumer / "b", f"-DCMAKE_CXX_COMPILER={CLANG}",
        f"-DCMAKE_PREFIX_PATH={prefix};/opt/rocm")
    run("cmake", "--build", consumer / "b")
    env = dict(os.environ, LD_LIBRARY_PATH=str(prefix / "lib"))
    out = subprocess.run([str(consumer / "b" / "consumer")], capture_output=True, text=True, env=env)
    assert out.returncode == 0 and out.stdout.split() == ["34359738368", "1"], (out.stdout, out.stderr)
