"""Write a synthetic sparse matrix in the engine's binary CSR format.

Command-line counterpart of the reference's scripts/gen_matrices.py
(main :104-138): the same flags and defaults, the same four patterns and the
same file layout (csr_write_binary_host; csr.cu:125-150 reads it back):

    int32 rows, int32 cols, int32 nnz, int32 row_ptr[rows+1],
    int32 col_idx[nnz], float32 values[nnz]     (little-endian)

The matrices come from the engine's own C++ generators (std::mt19937 seeded
with --seed), not numpy's stream, so the structure of each pattern matches the
reference's and the random draws do not:

    uniform         Bernoulli(density) per cell, values U[-1,1)
                    (generate_uniform_random_csr, csr.cu:74-103)
    banded          every cell with |r - c| <= bandwidth (gen_matrices.py:37-48)
    block-diagonal  floor(min(rows, cols) / block) dense blocks (:51-63)
    power-law       Pareto(alpha) + 1 degrees scaled to mean-deg, rounded,
                    clipped to [1, cols]; distinct uniform columns (:66-81)

Usage:
    python -m spmm_amd.gen_matrices --pattern banded --rows 4096 --cols 4096 \
        --bandwidth 32 --out data/banded_4096.bin
"""
from __future__ import annotations

import argparse
import os
import sys

from . import (csr_write_binary_host, generate_banded_csr,
               generate_block_diagonal_uniform_csr, generate_power_law_csr,
               generate_uniform_random_csr)

PATTERNS = ("uniform", "banded", "block-diagonal", "power-law")


def build(pattern: str, rows: int, cols: int, *, density: float = 0.01, bandwidth: int = 16,
          block: int = 32, mean_deg: float = 16.0, alpha: float = 2.5, seed: int = 42):
    """The host CSR of one pattern with the reference CLI's parameter meaning."""
    if pattern == "uniform":
        return generate_uniform_random_csr(rows, cols, density, seed)
    if pattern == "banded":
        return generate_banded_csr(rows, cols, bandwidth, seed)
    if pattern == "block-diagonal":
        return generate_block_diagonal_uniform_csr(rows, cols, block, seed)
    if pattern == "power-law":
        # gen_matrices.py clips degrees to [1, cols]: the cap is the width
        return generate_power_law_csr(rows, cols, mean_deg, alpha, max(1, cols), seed)
    raise ValueError(f"unknown pattern {pattern!r}; expected one of {', '.join(PATTERNS)}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m spmm_amd.gen_matrices", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--pattern", required=True, choices=PATTERNS)
    ap.add_argument("--rows", type=int, required=True)
    ap.add_argument("--cols", type=int, required=True)
    ap.add_argument("--density", type=float, default=0.01, help="for uniform")
    ap.add_argument("--bandwidth", type=int, default=16, help="for banded")
    ap.add_argument("--block", type=int, default=32, help="for block-diagonal")
    ap.add_argument("--mean-deg", type=float, default=16.0, help="for power-law")
    ap.add_argument("--alpha", type=float, default=2.5, help="for power-law")
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--out", required=True)
    a = ap.parse_args(argv)

    m = build(a.pattern, a.rows, a.cols, density=a.density, bandwidth=a.bandwidth,
              block=a.block, mean_deg=a.mean_deg, alpha=a.alpha, seed=a.seed)
    parent = os.path.dirname(os.path.abspath(a.out))
    os.makedirs(parent, exist_ok=True)
    csr_write_binary_host(m, a.out)
    cells = float(a.rows) * float(a.cols)
    density = m.nnz / cells if cells > 0 else 0.0
    print(f"wrote {a.out}  rows={a.rows} cols={a.cols} nnz={m.nnz} density={density:.6f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
