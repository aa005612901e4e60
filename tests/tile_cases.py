"""Random run-structured BSR inputs for the run-panel plan and kernel tests.

Block-row r holds a run of consecutive block-columns [s_r, s_r + L_r) (or
nothing), each block with 1-4 entries in distinct cells, on a matrix whose last
block-row and block-column may be partial.  `panels_contiguous` restates the
plan's acceptance rule: within each panel of R block-rows the runs of the
non-empty block-rows cover their union without a gap.
"""
from __future__ import annotations

import numpy as np


def random_runs(rng, block_rows: int, block_cols: int, step_max: int = 2,
                max_len: int = 12, p_empty: float = 0.1):
    runs, s = [], 0
    for _ in range(block_rows):
        if rng.random() < p_empty:
            runs.append((0, 0))
            continue
        s = min(block_cols - 1, s + int(rng.integers(0, step_max + 1)))
        runs.append((s, int(rng.integers(1, min(max_len, block_cols - s) + 1))))
    return runs


def csr_from_runs(S, rng, runs, M: int, K: int):
    rows, cols = [], []
    for br, (s, L) in enumerate(runs):
        for b in range(s, s + L):
            r0, c0 = br * 16, b * 16
            nr, nc = min(16, M - r0), min(16, K - c0)
            for cell in rng.choice(nr * nc, size=min(int(rng.integers(1, 5)), nr * nc),
                                   replace=False):  # distinct cells: no duplicate entries
                rows.append(r0 + int(cell) // nc)
                cols.append(c0 + int(cell) % nc)
    vals = rng.uniform(-1, 1, len(rows)).astype(np.float32)
    A = S.csr_from_coo_host(M, K, np.array(rows, np.int64), np.array(cols, np.int64), vals)
    A.values = S.round_to_fp16(A.values)
    return A


def panels_contiguous(runs, R: int) -> bool:
    for p in range(0, len(runs), R):
        cover = set()
        for s, L in runs[p:p + R]:
            cover.update(range(s, s + L))
        if cover and max(cover) - min(cover) + 1 != len(cover):
            return False
    return True


def random_case(S, rng):
    """(A, runs, M, K) with ragged M and K."""
    block_rows = int(rng.integers(1, 80))
    block_cols = int(rng.integers(1, 90))
    M = block_rows * 16 - int(rng.integers(0, 16))
    K = block_cols * 16 - int(rng.integers(0, 16))
    runs = random_runs(rng, block_rows, block_cols, step_max=int(rng.integers(0, 4)),
                       max_len=int(rng.choice([2, 5, 12, 40])))
    return csr_from_runs(S, rng, runs, M, K), runs, M, K
