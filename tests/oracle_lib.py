"""ctypes binding of the CPU oracle (oracle/build/liboracle.so) for the tests.

Test infrastructure only: the oracle checks the engine, it is never the thing
measured or shipped.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "build", "liboracle.so")

_lib = None
_P = ctypes.POINTER
_vp, _int, _long, _float, _double, _u32 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_long,
                                           ctypes.c_float, ctypes.c_double, ctypes.c_uint32)

_SIGS = {
    "oracle_mt_raw": (None, [_u32, _vp, _long]),
    "oracle_canonical_f32": (_float, [_u32]),
    "oracle_generate_uniform_csr": (_long, [_int, _int, _float, _int, _vp, _vp, _vp, _long]),
    "oracle_generate_dense": (None, [_int, _int, _int, _vp]),
    "oracle_coo_to_csr": (_int, [_int, _long, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oracle_csr_spmm_f64": (None, [_int, _int, _vp, _vp, _vp, _vp, _vp, _vp, _int]),
    "oracle_csr_spmm_f32_fma": (None, [_int, _int, _vp, _vp, _vp, _vp, _vp]),
    "oracle_f32_to_f16": (ctypes.c_uint16, [_float]),
    "oracle_f16_to_f32": (_float, [ctypes.c_uint16]),
    "oracle_f32_to_f16_array": (None, [_vp, _vp, _long]),
    "oracle_bsr_count": (_long, [_int, _int, _vp, _vp, _vp]),
    "oracle_bsr_fill": (_int, [_int, _int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oracle_bsr_stats": (None, [_int, _int, _long, _long, _P(_double), _P(_double), _P(_long)]),
    "oracle_bsr_spmm_f32": (None, [_int, _int, _int, _vp, _vp, _vp, _vp, _vp, _int]),
    "oracle_hybrid_rule": (_int, [_double, _int, _float, _P(_int)]),
    "oracle_nnz_balanced_bounds": (None, [_int, _vp, _int, _vp]),
    "oracle_compare": (None, [_vp, _vp, _long, _P(_float), _P(_float), _P(_float)]),
    "oracle_rel_l2": (_float, [_vp, _vp, _long]),
    "oracle_median": (_float, [_vp, _int]),
}


def build() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            build()
        h = ctypes.CDLL(ORACLE_LIB)
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data if a.size else 0


def mt_raw(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().oracle_mt_raw(seed, _p(out), n)
    return out


def canonical_f32(draw: int) -> float:
    return lib().oracle_canonical_f32(draw)


def uniform_csr(rows: int, cols: int, density: float, seed: int):
    """(row_ptr, col_idx, values) of csr.cu:74-103's generator."""
    rp = np.empty(rows + 1, dtype=np.int32)
    nnz = lib().oracle_generate_uniform_csr(rows, cols, density, seed, _p(rp), 0, 0, 0)
    ci = np.empty(max(nnz, 1), dtype=np.int32)
    va = np.empty(max(nnz, 1), dtype=np.float32)
    got = lib().oracle_generate_uniform_csr(rows, cols, density, seed, _p(rp), _p(ci), _p(va), nnz)
    assert got == nnz
    return rp, ci[:nnz], va[:nnz]


def uniform_nnz(rows: int, cols: int, density: float, seed: int) -> int:
    rp = np.empty(rows + 1, dtype=np.int32)
    return int(lib().oracle_generate_uniform_csr(rows, cols, density, seed, _p(rp), 0, 0, 0))


def dense(rows: int, cols: int, seed: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    lib().oracle_generate_dense(rows, cols, seed, _p(out))
    return out


def coo_to_csr(rows: int, r, c, v):
    r = np.ascontiguousarray(r, np.int32)
    c = np.ascontiguousarray(c, np.int32)
    v = np.ascontiguousarray(v, np.float32)
    rp = np.empty(rows + 1, np.int32)
    ci = np.empty(max(v.size, 1), np.int32)
    va = np.empty(max(v.size, 1), np.float32)
    rc = lib().oracle_coo_to_csr(rows, v.size, _p(r), _p(c), _p(v), _p(rp), _p(ci), _p(va))
    if rc != 0:
        raise ValueError(f"oracle_coo_to_csr failed ({rc})")
    return rp, ci[:v.size], va[:v.size]


def csr_spmm_f64(row_ptr, col_idx, values, B, threads: int = 1, with_abs: bool = True):
    """(C, |A||B|) in float64."""
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    col_idx = np.ascontiguousarray(col_idx, np.int32)
    values = np.ascontiguousarray(values, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M = row_ptr.size - 1
    N = B.shape[1]
    C = np.empty((M, N), np.float64)
    A = np.empty((M, N), np.float64) if with_abs else None
    lib().oracle_csr_spmm_f64(M, N, _p(row_ptr), _p(col_idx), _p(values), _p(B), _p(C),
                              _p(A) if A is not None else 0, threads)
    return C, A


def csr_spmm_f32_fma(row_ptr, col_idx, values, B):
    """The reference baseline kernel's fp32 fused chain (spmm_baseline.cu:11-25)."""
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    col_idx = np.ascontiguousarray(col_idx, np.int32)
    values = np.ascontiguousarray(values, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M = row_ptr.size - 1
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    lib().oracle_csr_spmm_f32_fma(M, N, _p(row_ptr), _p(col_idx), _p(values), _p(B), _p(C))
    return C


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h: int) -> float:
    return lib().oracle_f16_to_f32(h)


def bsr_build(M: int, K: int, row_ptr, col_idx, values):
    """(block_row_ptr, block_col_idx, block_values_fp16_bits)."""
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    col_idx = np.ascontiguousarray(col_idx, np.int32)
    values = np.ascontiguousarray(values, np.float32)
    brp = np.empty((M + 15) // 16 + 1, np.int32)
    nb = lib().oracle_bsr_count(M, K, _p(row_ptr), _p(col_idx), _p(brp))
    bci = np.empty(max(nb, 1), np.int32)
    bv = np.empty(max(nb, 1) * 256, np.uint16)
    rc = lib().oracle_bsr_fill(M, K, _p(row_ptr), _p(col_idx), _p(values), _p(brp), _p(bci), _p(bv))
    if rc != 0:
        raise ValueError("oracle_bsr_fill: column out of range")
    return brp, bci[:nb], bv[:nb * 256]


def bsr_stats(M: int, K: int, num_blocks: int, nnz: int):
    fill, dens, stored = ctypes.c_double(), ctypes.c_double(), ctypes.c_long()
    lib().oracle_bsr_stats(M, K, num_blocks, nnz, ctypes.byref(fill), ctypes.byref(dens),
                           ctypes.byref(stored))
    return fill.value, dens.value, stored.value


def bsr_spmm_f32(M: int, K: int, brp, bci, bv, B16, threads: int = 1) -> np.ndarray:
    B16 = np.ascontiguousarray(B16, np.uint16)
    N = B16.shape[1]
    C = np.empty((M, N), np.float32)
    lib().oracle_bsr_spmm_f32(M, K, N, _p(np.ascontiguousarray(brp, np.int32)),
                              _p(np.ascontiguousarray(bci, np.int32)),
                              _p(np.ascontiguousarray(bv, np.uint16)), _p(B16), _p(C), threads)
    return C


def hybrid_rule(fill: float, N: int, threshold: float):
    why = ctypes.c_int()
    use = lib().oracle_hybrid_rule(fill, N, threshold, ctypes.byref(why))
    return use, why.value


def nnz_balanced_bounds(row_ptr, parts: int) -> np.ndarray:
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    out = np.empty(parts + 1, np.int32)
    lib().oracle_nnz_balanced_bounds(row_ptr.size - 1, _p(row_ptr), parts, _p(out))
    return out


def compare(ours, ref):
    a = np.ascontiguousarray(ours, np.float32).ravel()
    b = np.ascontiguousarray(ref, np.float32).ravel()
    ma, mr, rl = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
    lib().oracle_compare(_p(a), _p(b), a.size, ctypes.byref(ma), ctypes.byref(mr), ctypes.byref(rl))
    return ma.value, mr.value, rl.value


def rel_l2(ours, ref) -> float:
    a = np.ascontiguousarray(ours, np.float32).ravel()
    b = np.ascontiguousarray(ref, np.float32).ravel()
    return lib().oracle_rel_l2(_p(a), _p(b), a.size)


def median(v) -> float:
    a = np.ascontiguousarray(v, np.float32).copy()
    return lib().oracle_median(_p(a), a.size)
