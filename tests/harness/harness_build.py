"""Build the C++ harness (tests/harness/bench_flash_attention) against
include/flash_attention.h, libfa_mi355x.so and the oracle checker.

Run by __graft_entry__.build() after both libraries exist. The binary finds
them through $ORIGIN-relative run paths, so it works wherever the tree is
copied. Test infrastructure, not part of the product.
"""
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
BINARY = os.path.join(HERE, "bench_flash_attention")


def build(verbose: bool = False) -> str:
    hipcc = next(c for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")) if c and os.path.exists(c))
    cmd = [
        hipcc, "-std=c++17", "-O2", "-Wall",
        f"-I{os.path.join(REPO, 'include')}", f"-I{os.path.join(REPO, 'oracle')}",
        os.path.join(HERE, "bench_flash_attention.cpp"), "-o", BINARY + ".tmp",
        f"-L{os.path.join(REPO, 'cuda_fused_attention_amd')}", "-lfa_mi355x",
        f"-L{os.path.join(REPO, 'oracle')}", "-loracle",
        "-Wl,-rpath,$ORIGIN/../../cuda_fused_attention_amd:$ORIGIN/../../oracle",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(BINARY + ".tmp", BINARY)
    return BINARY


if __name__ == "__main__":
    print(build(verbose=True))
