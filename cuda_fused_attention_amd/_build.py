"""In-tree build of libfa_mi355x.so for gfx950 with hipcc (no JIT cache, no
site-packages install): the built library sits next to this file and travels
with the source tree."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libfa_mi355x.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

SOURCES = ["fa_unfused.hip", "fa_fused.hip", "fa_calib.hip", "fa_api.cpp"]

# -packed-fp32-ops: the compiler must not form v_pk_{add,mul,fma}_f32 by
# itself from float code (those forms have miscomputed on this pool).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # kernel arguments preloaded into SGPRs by the command processor: a
    # launch's waves start without the scalar loads of the argument block
    # (1-1.6 % on the (2,8,2048,D) shapes, 5 % on small grids; the compiler
    # keeps a loading entry for firmware without preloading)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfa_mi355x.so)")


def _compile(cc: str, src: str, obj: str, extra, verbose: bool) -> str:
    cmd = [cc, *HIP_FLAGS, f"-I{CSRC}", *extra, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stderr)
        raise subprocess.CalledProcessError(proc.returncode, cmd)
    if verbose and proc.stderr:
        sys.stderr.write(proc.stderr)
    return proc.stderr


def build(verbose: bool = False) -> str:
    """Compile every source for gfx950 and link libfa_mi355x.so in-tree.

    fa_fused.hip is compiled with the compiler's kernel resource report on;
    kernel_resources.py turns it into the table the resource query reads
    (AGPRs and SGPRs per kernel), compiled in as one more source."""
    from . import kernel_resources

    out_dir = os.path.join(PKG_DIR, "_build")
    os.makedirs(out_dir, exist_ok=True)
    cc = hipcc()
    jobs = []
    for src in SOURCES:
        obj = os.path.join(out_dir, os.path.splitext(src)[0] + ".o")
        extra = ["-x", "hip"]
        if src == "fa_fused.hip":
            extra.append("-Rpass-analysis=kernel-resource-usage")
        jobs.append((os.path.join(CSRC, src), obj, extra))
    with ThreadPoolExecutor(max_workers=len(jobs)) as pool:
        remarks = list(pool.map(lambda j: _compile(cc, j[0], j[1], j[2], verbose), jobs))
    entries = kernel_resources.parse(remarks[SOURCES.index("fa_fused.hip")])
    if not entries:
        raise RuntimeError("the compiler reported no resources for the fused kernels")
    table_src = os.path.join(out_dir, "fa_kernel_resources.cpp")
    kernel_resources.write(entries, table_src)
    table_obj = os.path.join(out_dir, "fa_kernel_resources.o")
    _compile(cc, table_src, table_obj, ["-x", "hip"], verbose)
    objs = [j[1] for j in jobs] + [table_obj]
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB_PATH)
