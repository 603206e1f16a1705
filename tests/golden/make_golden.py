"""Extract the reference's published formula scores into a JSON fixture.

Reads the A100 evaluation CSVs of the reference (data files, not code) and
writes tests/golden/formula_scores.json:

  gemm_three_ops_formula_summary.csv   op, M, N, K, top-1 config, score (78 rows)
  conv2d_formula_changed_after_costmodel.csv   shape, top-1 config, score (9 rows)

Run once where /root/reference exists:  python tests/golden/make_golden.py
"""

import csv
import json
from pathlib import Path

REF = Path("/root/reference/evaluation")
OUT = Path(__file__).resolve().parent / "formula_scores.json"


def main():
    gemm_rows = []
    with open(REF / "gemm_three_ops_formula_summary.csv") as f:
        for r in csv.DictReader(f):
            gemm_rows.append({"op": r["op"], "M": int(r["M"]), "N": int(r["N"]), "K": int(r["K"]),
                              "config": r["config"], "score": float(r["score"])})
    conv_rows = []
    with open(REF / "conv2d_formula_changed_after_costmodel.csv") as f:
        for r in csv.DictReader(f):
            conv_rows.append({"N": int(r["N"]), "C": int(r["C"]), "H": int(r["H"]), "W": int(r["W"]),
                              "F": int(r["F_out"]), "KH": int(r["Kernel_H"]), "KW": int(r["Kernel_W"]),
                              "stride": int(r["Stride"]), "pad": int(r["Pad"]),
                              "config": r["Formula_Config"], "score": float(r["Formula_Score"])})
    OUT.write_text(json.dumps({
        "source": "reference evaluation/gemm_three_ops_formula_summary.csv, "
                  "evaluation/conv2d_formula_changed_after_costmodel.csv (A100 GPUSpec)",
        "gemm": gemm_rows, "conv2d": conv_rows}, indent=1))
    print(f"wrote {OUT} ({len(gemm_rows)} gemm rows, {len(conv_rows)} conv rows)")


if __name__ == "__main__":
    main()
