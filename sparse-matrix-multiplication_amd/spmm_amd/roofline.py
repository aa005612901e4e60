"""MI355X roofline analysis of SpMM benchmark lines.

Counterpart of the reference's scripts/roofline.py (parse :157-174,
csr_dram_bytes :177-185, analyse :188-212, main :228-268, plot :271-309),
with MI355X ceilings in place of the T4's and the BSR byte model added for
the matrix-core kernel.  It reads the ``kernel=...`` lines that
``spmm_bench`` prints (or the CSV of ``run_pattern_sweep``) and computes,
for every kernel x problem cell:

  * achieved GFLOP/s            2*nnz*N / time (as printed)
  * compulsory HBM bytes        every operand read or written once
  * arithmetic intensity (AI)   FLOPs / compulsory bytes
  * roofline ceiling            min(compute peak, AI * HBM peak)
  * % of the ceiling, % of HBM peak, and for the MFMA kernel % of the fp16
    MFMA peak on the executed FLOPs (2*256*blocks*N)
  * optionally (--gather-tbs) the CSR gather roof: every nonzero pulls its
    B row segment (N*4 bytes) through the CU's vector-memory path, which
    bounds uniform-random inputs long before HBM does.

Byte models (fp32 CSR, fp16 BSR with 16x16 blocks):
  CSR  8*nnz + 4*(M+1) + 4*K*N + 4*M*N                   (roofline.py:177-185)
  BSR  512*blocks + 4*blocks + 4*(M/16+1) + 2*K*N + 4*M*N

The block count of an MFMA row comes from the ``bsr_stats blocks=`` line
``spmm_bench`` prints before it; a row without one falls back to nnz/256
blocks (fill-in 1.0) and is marked ``blocks_estimated``.

Usage:
    spmm_bench --kernel all ... > log.txt
    python -m spmm_amd.roofline log.txt [--csv roofline.csv] [--plot roofline.png]
                                        [--gather-tbs 39.3]
"""
from __future__ import annotations

import argparse
import csv
import os
import re
import sys
from typing import Dict, Iterable, List, Optional

# MI355X datasheet peaks
HBM_GBS = 8000.0               # HBM3E, GB/s
FP32_GFLOPS = 157300.0         # vector fp32 (packed), GFLOP/s
MFMA_F16_GFLOPS = 2516600.0    # dense fp16 matrix cores, GFLOP/s
L2_BYTES = 4 * 1024 * 1024     # per XCD
RIDGE_FP32 = FP32_GFLOPS / HBM_GBS

FIELD = re.compile(r"(\w+)=(\"[^\"]*\"|[^\s]+)")
CSV_INT = ("m", "k", "n", "nnz")
CSV_FLOAT = ("time_ms", "gflops")


def _fields(line: str) -> Dict[str, str]:
    return {k: v.strip('"') for k, v in FIELD.findall(line)}


def parse(text: str) -> List[dict]:
    """kernel= lines of spmm_bench output; a bsr_stats line attaches its block
    count to the following wmma line (as spmm_bench prints them)."""
    rows: List[dict] = []
    blocks: Optional[int] = None
    for raw in text.splitlines():
        line = raw.strip()
        if line.startswith("bsr_stats"):
            d = _fields(line)
            blocks = int(d["blocks"]) if "blocks" in d else None
            continue
        if not line.startswith("kernel="):
            continue
        d = _fields(line)
        row = {"kernel": d["kernel"], "m": int(d["m"]), "k": int(d["k"]), "n": int(d["n"]),
               "nnz": int(d["nnz"]), "time_ms": float(d["time_ms"]),
               "gflops": float(d["gflops"]), "blocks": None}
        if _is_mfma(row["kernel"]) and blocks is not None:
            row["blocks"] = blocks
        rows.append(row)
    return rows


def parse_sweep_csv(path: str) -> List[dict]:
    """Rows of run_pattern_sweep's CSV (pattern,kernel,m,k,n,nnz,density,time_ms,gflops)."""
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            row = {"kernel": r["kernel"], "blocks": None, "pattern": r.get("pattern", "")}
            for c in CSV_INT:
                row[c] = int(r[c])
            for c in CSV_FLOAT:
                row[c] = float(r[c])
            rows.append(row)
    return rows


def _is_mfma(kernel: str) -> bool:
    return kernel == "wmma" or kernel == "hybrid[wmma]"


def csr_bytes(m: int, k: int, n: int, nnz: int) -> float:
    """Compulsory HBM bytes of a fp32 CSR SpMM (roofline.py:177-185)."""
    return 8.0 * nnz + 4.0 * (m + 1) + 4.0 * k * n + 4.0 * m * n


def bsr_bytes(m: int, k: int, n: int, blocks: int) -> float:
    """Compulsory HBM bytes of a 16x16 fp16 BSR SpMM with fp32 C."""
    return 516.0 * blocks + 4.0 * ((m + 15) // 16 + 1) + 2.0 * k * n + 4.0 * m * n


def analyse(rows: Iterable[dict], gather_tbs: Optional[float] = None) -> List[dict]:
    out = []
    for r in rows:
        m, k, n, nnz = r["m"], r["k"], r["n"], r["nnz"]
        flops = 2.0 * nnz * n
        ach = r["gflops"]
        res = dict(r)
        if _is_mfma(r["kernel"]):
            est = r.get("blocks") is None
            blocks = (nnz + 255) // 256 if est else r["blocks"]
            bytes_ = bsr_bytes(m, k, n, blocks)
            exec_flops = 2.0 * 256.0 * blocks * n
            ai = flops / bytes_
            ceiling = min(MFMA_F16_GFLOPS * flops / max(exec_flops, 1.0), ai * HBM_GBS)
            t_s = r["time_ms"] * 1.0e-3
            res.update(blocks=blocks, blocks_estimated=est, exec_flops=exec_flops,
                       pct_compute_peak=100.0 * exec_flops / t_s / 1e9 / MFMA_F16_GFLOPS
                       if t_s > 0 else 0.0,
                       bound="mfma" if ai * HBM_GBS > MFMA_F16_GFLOPS * flops / max(exec_flops, 1.0)
                       else "hbm")
        else:
            bytes_ = csr_bytes(m, k, n, nnz)
            ai = flops / bytes_
            ceiling = min(FP32_GFLOPS, ai * HBM_GBS)
            res.update(blocks_estimated=False, exec_flops=flops,
                       pct_compute_peak=100.0 * ach / FP32_GFLOPS,
                       bound="fp32" if ai > RIDGE_FP32 else "hbm")
            if gather_tbs:
                gather_bytes = 4.0 * nnz * n
                # GFLOP/s the gather path allows: FLOPs per gathered byte x rate
                res["gather_ceiling_gflops"] = flops / gather_bytes * gather_tbs * 1000.0
                res["pct_gather_roof"] = 100.0 * ach / res["gather_ceiling_gflops"]
        eff_bw = bytes_ / (r["time_ms"] * 1.0e6) if r["time_ms"] > 0 else 0.0
        res.update(flops=flops, hbm_bytes=bytes_, ai_flop_per_byte=ai, ceiling_gflops=ceiling,
                   pct_roofline=100.0 * ach / ceiling if ceiling > 0 else 0.0,
                   eff_hbm_gbs=eff_bw, pct_hbm=100.0 * eff_bw / HBM_GBS,
                   B_fits_L2=(k * n * (2 if _is_mfma(r["kernel"]) else 4)) <= L2_BYTES)
        out.append(res)
    return out


COLUMNS = ["kernel", "m", "k", "n", "nnz", "blocks", "time_ms", "gflops", "hbm_bytes",
           "ai_flop_per_byte", "ceiling_gflops", "pct_roofline", "eff_hbm_gbs", "pct_hbm",
           "pct_compute_peak", "bound", "B_fits_L2", "blocks_estimated",
           "gather_ceiling_gflops", "pct_gather_roof"]


def write_csv(path: str, rows: List[dict]) -> None:
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLUMNS, extrasaction="ignore")
        w.writeheader()
        for r in rows:
            w.writerow(r)


def table(res: List[dict]) -> str:
    """Console table: per problem cell, the best CSR kernel and the MFMA kernel."""
    lines = [f"MI355X ceilings: HBM {HBM_GBS:.0f} GB/s | fp32 {FP32_GFLOPS:.0f} GFLOP/s | "
             f"fp16 MFMA {MFMA_F16_GFLOPS:.0f} GFLOP/s | fp32 ridge {RIDGE_FP32:.1f} FLOP/byte", ""]
    hdr = (f"{'cell (m, k, n, nnz)':>30} {'kernel':>14} {'AI':>7} {'roof G':>9} "
           f"{'GFLOP/s':>9} {'%roof':>6} {'%HBM':>6} {'%peak':>6}")
    lines += [hdr, "-" * len(hdr)]
    cells = sorted({(r["m"], r["k"], r["n"], r["nnz"]) for r in res})
    for cell in cells:
        group = [r for r in res if (r["m"], r["k"], r["n"], r["nnz"]) == cell]
        csr = [r for r in group if not _is_mfma(r["kernel"])]
        picks = ([max(csr, key=lambda r: r["gflops"])] if csr else []) + \
                [r for r in group if _is_mfma(r["kernel"])]
        for r in picks:
            lines.append(f"{'%d, %d, %d, %d' % cell:>30} {r['kernel']:>14} "
                         f"{r['ai_flop_per_byte']:>7.1f} {r['ceiling_gflops']:>9.0f} "
                         f"{r['gflops']:>9.1f} {r['pct_roofline']:>5.1f}% {r['pct_hbm']:>5.1f}% "
                         f"{r['pct_compute_peak']:>5.2f}%")
    return "\n".join(lines)


def plot(res: List[dict], path: str, gather_tbs: Optional[float] = None) -> bool:
    try:
        import matplotlib
        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
        import numpy as np
    except ImportError:
        print("matplotlib not available; skipping plot", file=sys.stderr)
        return False
    fig, ax = plt.subplots(figsize=(8, 6))
    ai = np.logspace(-1, 3.5, 200)
    ax.plot(ai, np.minimum(FP32_GFLOPS, ai * HBM_GBS), "k-", lw=2, label="fp32 roofline (HBM)")
    ax.plot(ai, np.minimum(MFMA_F16_GFLOPS, ai * HBM_GBS), "k--", lw=1,
            label="fp16 MFMA roofline (HBM)")
    if gather_tbs:
        # 2 FLOPs per gathered fp32 B element: 0.5 FLOP per byte through the CUs
        ax.axhline(0.5 * gather_tbs * 1000.0, c="tab:blue", ls=":", lw=1.5,
                   label=f"CSR gather roof ({gather_tbs:g} TB/s into the CUs)")
    for r in res:
        mfma = _is_mfma(r["kernel"])
        ax.plot(r["ai_flop_per_byte"], r["gflops"], "s" if mfma else "o", ms=6,
                c="tab:red" if mfma else "tab:blue")
        ax.annotate(f"{r['kernel']}\nm={r['m']} n={r['n']}", (r["ai_flop_per_byte"], r["gflops"]),
                    fontsize=5, xytext=(3, 3), textcoords="offset points")
    ax.set_xscale("log")
    ax.set_yscale("log")
    ax.set_xlabel("Arithmetic intensity (FLOP/byte, compulsory HBM bytes)")
    ax.set_ylabel("GFLOP/s")
    ax.set_title("MI355X roofline: SpMM kernels (o CSR fp32, s BSR fp16 MFMA)")
    ax.legend(loc="lower right", fontsize=8)
    ax.grid(True, which="both", ls=":", alpha=0.4)
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    fig.tight_layout()
    fig.savefig(path, dpi=130)
    plt.close(fig)
    return True


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("input", help="spmm_bench output (kernel= lines) or run_pattern_sweep CSV")
    ap.add_argument("--csv", default=None, help="write the roofline table as CSV")
    ap.add_argument("--plot", default=None, help="write a roofline PNG")
    ap.add_argument("--gather-tbs", type=float, default=None,
                    help="CU gather rate in TB/s for the CSR gather roof "
                         "(64 B/clk x 256 CUs x 2.4 GHz = 39.3)")
    args = ap.parse_args(argv)
    if args.input.endswith(".csv"):
        rows = parse_sweep_csv(args.input)
    else:
        with open(args.input) as f:
            rows = parse(f.read())
    if not rows:
        print(f"no kernel= lines in {args.input}", file=sys.stderr)
        return 1
    res = analyse(rows, args.gather_tbs)
    print(table(res))
    if args.csv:
        write_csv(args.csv, res)
        print(f"\nwrote {args.csv}")
    if args.plot and plot(res, args.plot, args.gather_tbs):
        print(f"wrote {args.plot}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
