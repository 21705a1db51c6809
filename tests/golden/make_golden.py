"""Writes tests/golden/c1_uniform_dense.npz
(B=1, H=2, N=128, D=64, dense, Q/K/V uniform[-1,1) bf16 from seeds 11/22/33)
with the SHA-256 of each input's bf16 bytes and the FP64 oracle output.

Run from the repository root:  python tests/golden/make_golden.py
The reference's path is CUDA and cannot run here; the fixture is produced by
this repository's oracle (oracle/oracle.cpp), which tests/test_oracle_pins.py
pins against the reference's published statistics, and it then guards both
the generator and the oracle against regressions."""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

B, H, N, D = 1, 2, 128, 64


def main():
    q, k, v = oracle.make_inputs(B, H, N, D, "uniform")
    o_ref = oracle.attention(q, k, v, False)
    sha = {name: hashlib.sha256(arr.tobytes()).hexdigest() for name, arr in (("q", q), ("k", k), ("v", v))}
    path = os.path.join(ROOT, "tests", "golden", "c1_uniform_dense.npz")
    np.savez_compressed(path, shape=np.array([B, H, N, D]), seeds=np.array([11, 22, 33]),
                        sha_q=sha["q"], sha_k=sha["k"], sha_v=sha["v"], o_ref=o_ref)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
