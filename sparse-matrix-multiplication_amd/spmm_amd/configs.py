"""The five BASELINE configurations (c1 .. c5) as engine-generated inputs.

Seeds: the uniform configs use A seed 42 and B seed 43 (seed + 1), as the
reference harness does (harness.cu:304); the structured configs use fixed
seeds of their own.  Patterns follow gen_matrices.py:37-81 with the values the
BASELINE text names (block-diagonal N(0,1)*0.1, power-law capped at 4096).
The fp16 configs (c3, c4) round A's values and B to fp16 on the host, so the
fp32 and fp16 views of an operand hold the same numbers.
"""
from __future__ import annotations

import numpy as np

# name: (pattern, M (= K), N, fp16 operands, one-line description)
CONFIGS = {
    "c1": ("uniform", 4096, 128, False,
           "uniform-random CSR 4096x4096 density 0.01, B 4096x128 fp32"),
    "c2": ("uniform", 8192, 128, False,
           "uniform-random CSR 8192x8192 density 0.01, B 8192x128 fp32"),
    "c3": ("banded", 8192, 128, True,
           "banded 8192x8192 half-bandwidth 64 as BSR 16x16 fp16, B 8192x128 fp16"),
    "c4": ("block_diagonal", 8192, 256, True,
           "block-diagonal 32 x 256^2 as BSR 16x16 fp16, B 8192x256 fp16"),
    "c5": ("power_law", 16384, 128, False,
           "power-law 16384x16384 (Pareto 1.5, mean 164, cap 4096), B 16384x128 fp32"),
}


def make_config(S, name: str):
    """(HostCSR, B float32 K x N) of one BASELINE config.  S is the spmm_amd
    module (passed in so this file imports nothing that loads the library)."""
    pattern, M, N, fp16, _ = CONFIGS[name]
    if pattern == "uniform":
        A = S.generate_uniform_random_csr(M, M, 0.01, 42)
        B = S.generate_dense_row_major(M, N, 43)
    elif pattern == "banded":
        A = S.generate_banded_csr(M, M, 64, 1003)
        B = S.generate_dense_row_major(M, N, 1004)
    elif pattern == "block_diagonal":
        A = S.generate_block_diagonal_csr(M, M, 256, 2003, 0.1)
        B = S.generate_dense_row_major(M, N, 2004)
    else:
        A = S.generate_power_law_csr(M, M, 164.0, 1.5, 4096, 3003)
        B = S.generate_dense_row_major(M, N, 3004)
    if fp16:
        A.values = S.round_to_fp16(A.values)
        B = S.round_to_fp16(B)
    return A, np.ascontiguousarray(B, dtype=np.float32)
