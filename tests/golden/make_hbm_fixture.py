"""Writes tests/golden/reference_hbm_model.json: the `algorithmic_hbm_gb`
column of the reference's published results/raw/flash_attention/summary.csv
for the kernels whose byte model the oracle restates:

  v0_unfused       qkvo_bytes + unfused_score_bytes
                   (benchmarks/bench_flash_attention.cu:221-231,644)
  v2a_fused_tiled  the blocked K/V model with 8 query rows and 64-key tiles
  v2b_fused_tiled  (kernels/v2/v2a_tiled_pipelined.cu:480-503, and v2b's copy)
  v3_tensorcore    the same model with 64 query rows and 64-key (head_dim 64)
                   or 32-key (head_dim 128) tiles
                   (kernels/v3/v3_tensorcore.cu:146,795-818)

Data only: the shape, the mask, the published value (as the CSV text, so no
digit is lost) and the CSV line it came from. Run from the repository root
in the container that holds the reference:

    python tests/golden/make_hbm_fixture.py
"""
import csv
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
SOURCE = "/root/reference/results/raw/flash_attention/summary.csv"
KERNELS = ("v0_unfused", "v2a_fused_tiled", "v2b_fused_tiled", "v3_tensorcore")


def main():
    rows = []
    with open(SOURCE, newline="") as fh:
        reader = csv.DictReader(fh)
        for line_no, rec in enumerate(reader, start=2):
            if rec["kernel"] not in KERNELS:
                continue
            rows.append({
                "kernel": rec["kernel"],
                "batch": int(rec["batch"]), "heads": int(rec["heads"]), "seq_len": int(rec["seq_len"]),
                "head_dim": int(rec["head_dim"]), "causal": int(rec["causal"]),
                "algorithmic_hbm_gb": rec["algorithmic_hbm_gb"],
                "line": line_no,
            })
    out = {
        "source": "RichterWang/cuda_fused_attention results/raw/flash_attention/summary.csv "
                  "(column algorithmic_hbm_gb, written by benchmarks/bench_flash_attention.cu:641-648)",
        "rows": rows,
    }
    path = os.path.join(ROOT, "tests", "golden", "reference_hbm_model.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=0)
        fh.write("\n")
    print(path, len(rows), "rows")


if __name__ == "__main__":
    main()
