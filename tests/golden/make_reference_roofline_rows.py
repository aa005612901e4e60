"""Writes reference_roofline_rows.csv: the reference's committed sweep rows
(reports/data/sweep.csv: kernel, m, k, n, nnz, time_ms, gflops) joined row by
row with the two hardware-independent columns its roofline script computed
from them (reports/data/roofline.csv: ai_flop_per_byte, eff_dram_bw_gbs).

Data extraction only (no reference code runs).  Run in a checkout that has the
reference at /root/reference:

    python tests/golden/make_reference_roofline_rows.py
"""
import csv
import os
import sys

REF = "/root/reference/reports/data"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_roofline_rows.csv")


def main() -> int:
    with open(os.path.join(REF, "sweep.csv"), newline="") as f:
        sweep = list(csv.DictReader(f))
    with open(os.path.join(REF, "roofline.csv"), newline="") as f:
        roof = list(csv.DictReader(f))
    if len(sweep) != len(roof):
        print("row counts differ", len(sweep), len(roof), file=sys.stderr)
        return 1
    cols = ["kernel", "m", "k", "n", "nnz", "time_ms", "gflops", "ai_flop_per_byte",
            "eff_dram_bw_gbs"]
    with open(OUT, "w", newline="") as f:
        w = csv.writer(f, lineterminator="\n")
        w.writerow(cols)
        for s, r in zip(sweep, roof):
            same = (s["kernel"], s["m"], s["nnz"]) == (r["kernel"], r["m"], r["nnz"])
            if not same or float(s["gflops"]) != float(r["gflops"]):
                print("rows do not line up:", s, r, file=sys.stderr)
                return 1
            w.writerow([s["kernel"], s["m"], s["k"], s["n"], s["nnz"], s["time_ms"],
                        s["gflops"], r["ai_flop_per_byte"], r["eff_dram_bw_gbs"]])
    print(f"wrote {OUT} ({len(sweep)} rows)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
