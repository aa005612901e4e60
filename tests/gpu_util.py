"""Shared helpers of the GPU parity tests: config builders and the tolerance
checks (the oracle is the reference side of every comparison)."""
from __future__ import annotations

import numpy as np

from spmm_amd.configs import CONFIGS, make_config  # noqa: F401  (the five BASELINE configs)


def check_csr(C_gpu: np.ndarray, C64: np.ndarray, absC: np.ndarray, tol: float = 1e-5) -> float:
    """FP32 CSR bar: every element within tol * (|A||B|)_ij of the fp64 result,
    and the normwise error ||C - C64|| / ||C64|| within tol.  |A||B| is the
    scale of the rounding error of any fp32 summation order, so the bar does
    not break on cancellation.  Returns the relative L2 error."""
    C_gpu = np.asarray(C_gpu, dtype=np.float64)
    assert C_gpu.shape == C64.shape
    assert np.all(np.isfinite(C_gpu))
    err = np.abs(C_gpu - C64)
    bad = err > tol * absC
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"element {tuple(i)}: gpu={C_gpu[tuple(i)]!r} ref={C64[tuple(i)]!r} "
                             f"|A||B|={absC[tuple(i)]!r} ({int(bad.sum())} elements out of bound)")
    den = np.linalg.norm(C64)
    rel = float(np.linalg.norm(C_gpu - C64) / den) if den > 0 else float(np.linalg.norm(C_gpu))
    assert rel <= tol, rel
    return rel


def check_bsr(C_gpu: np.ndarray, C32: np.ndarray, absC: np.ndarray, tol: float = 1e-2) -> float:
    """FP16-input BSR bar: within tol of the oracle's fp32 accumulation of the
    same fp16 operands, elementwise relative to |A16||B16| and normwise."""
    C_gpu = np.asarray(C_gpu, dtype=np.float64)
    C32 = np.asarray(C32, dtype=np.float64)
    assert C_gpu.shape == C32.shape
    assert np.all(np.isfinite(C_gpu))
    err = np.abs(C_gpu - C32)
    bad = err > tol * absC
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"element {tuple(i)}: gpu={C_gpu[tuple(i)]!r} ref={C32[tuple(i)]!r} "
                             f"({int(bad.sum())} out of bound)")
    den = np.linalg.norm(C32)
    rel = float(np.linalg.norm(C_gpu - C32) / den) if den > 0 else float(np.linalg.norm(C_gpu))
    assert rel <= tol, rel
    return rel
