"""Python binding of the MI355X SpMM engine (ctypes over include/spmm_capi.h).

Mirrors the reference's C++ API for the hot path (reference src/csr.h,
src/bsr.h, src/kernels/*.h, src/spmm_hybrid.h): the same names, argument
meaning and failure conditions, raised as ``SpmmError`` instead of exiting.

Device buffers are torch tensors on ``cuda`` (torch is only the allocator and
the stream handle); every launch goes through ``libspmm_amd.so``.  When the
library is missing this module raises on first use -- there is no CPU
fallback for any device entry point.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "build", "libspmm_amd.so")

SPMM_OK, SPMM_INVALID, SPMM_UNSUPPORTED, SPMM_HIP_ERROR, SPMM_IO_ERROR, SPMM_NO_MEMORY = range(6)
BACKEND_CSR, BACKEND_WMMA = 0, 1

# kernel ids of spmm_c_launch_repeat / spmm_c_time_repeat
KERNEL_IDS = {
    "baseline": 0, "memopt": 1, "memopt_v2": 2, "tiled": 3,
    "tiled_v2": 4, "tiled_v3": 5, "tiled_v4": 6, "wmma": 7,
}
CSR_KERNELS = ("baseline", "memopt", "memopt_v2", "tiled", "tiled_v2", "tiled_v3", "tiled_v4")


class SpmmError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class CsrT(ctypes.Structure):
    _fields_ = [("num_rows", ctypes.c_int), ("num_cols", ctypes.c_int), ("nnz", ctypes.c_int),
                ("row_ptr", ctypes.c_void_p), ("col_idx", ctypes.c_void_p),
                ("values", ctypes.c_void_p)]


class BsrT(ctypes.Structure):
    _fields_ = [("num_rows", ctypes.c_int), ("num_cols", ctypes.c_int),
                ("block_rows", ctypes.c_int), ("block_cols", ctypes.c_int),
                ("num_blocks", ctypes.c_int), ("nnz", ctypes.c_int),
                ("row_ptr", ctypes.c_void_p), ("col_idx", ctypes.c_void_p),
                ("values", ctypes.c_void_p)]


class BsrStatsT(ctypes.Structure):
    _fields_ = [("num_blocks", ctypes.c_int), ("stored_elements", ctypes.c_long),
                ("original_nnz", ctypes.c_int), ("fill_in_ratio", ctypes.c_double),
                ("block_density", ctypes.c_double)]


class HybridPlanT(ctypes.Structure):
    _fields_ = [("backend", ctypes.c_int), ("fill_in_ratio", ctypes.c_double),
                ("block_density", ctypes.c_double), ("threshold", ctypes.c_float),
                ("n_aligned", ctypes.c_int), ("reason", ctypes.c_char_p)]


class EngineOptsT(ctypes.Structure):
    _fields_ = [("vec", ctypes.c_int), ("waves", ctypes.c_int), ("unroll", ctypes.c_int),
                ("rows_per_block", ctypes.c_int), ("groups", ctypes.c_int),
                ("slices", ctypes.c_int), ("global_loads", ctypes.c_int),
                ("row_groups", ctypes.c_int), ("entry_lanes", ctypes.c_int),
                ("max_row_hint", ctypes.c_int)]


class BsrOptsT(ctypes.Structure):
    _fields_ = [("row_group", ctypes.c_int), ("tiles", ctypes.c_int), ("per_wave", ctypes.c_int),
                ("depth", ctypes.c_int), ("xcd_order", ctypes.c_int),
                ("reserved0", ctypes.c_int), ("reserved1", ctypes.c_int),
                ("addressing", ctypes.c_int)]


_P = ctypes.POINTER
_vp, _int, _long, _float, _double = (ctypes.c_void_p, ctypes.c_int, ctypes.c_long,
                                     ctypes.c_float, ctypes.c_double)

# name -> (restype, argtypes)
_SIGNATURES = {
    "spmm_c_last_error": (ctypes.c_char_p, []),
    "spmm_c_version": (ctypes.c_char_p, []),
    "spmm_c_csr_alloc_host": (_int, [_int, _int, _int, _P(CsrT)]),
    "spmm_c_csr_free_host": (None, [_P(CsrT)]),
    "spmm_c_csr_from_coo_host": (_int, [_int, _int, _int, _vp, _vp, _vp, _P(CsrT)]),
    "spmm_c_generate_uniform_random_csr": (_int, [_int, _int, _float, _int, _P(CsrT)]),
    "spmm_c_csr_row_slice_host": (_int, [_P(CsrT), _int, _int, _P(CsrT)]),
    "spmm_c_csr_read_binary_host": (_int, [ctypes.c_char_p, _P(CsrT)]),
    "spmm_c_csr_write_binary_host": (_int, [_P(CsrT), ctypes.c_char_p]),
    "spmm_c_csr_to_device": (_int, [_P(CsrT), _P(CsrT)]),
    "spmm_c_csr_free_device": (_int, [_P(CsrT)]),
    "spmm_c_bsr_from_csr_host": (_int, [_P(CsrT), _P(BsrT)]),
    "spmm_c_bsr_free_host": (None, [_P(BsrT)]),
    "spmm_c_bsr_to_device": (_int, [_P(BsrT), _P(BsrT)]),
    "spmm_c_bsr_free_device": (_int, [_P(BsrT)]),
    "spmm_c_bsr_compute_stats": (_int, [_P(BsrT), _P(BsrStatsT)]),
    "spmm_c_generate_dense_row_major": (_int, [_int, _int, _int, _vp]),
    "spmm_c_generate_banded_csr": (_int, [_int, _int, _int, _int, _P(CsrT)]),
    "spmm_c_generate_block_diagonal_csr": (_int, [_int, _int, _int, _int, _float, _P(CsrT)]),
    "spmm_c_generate_block_diagonal_uniform_csr": (_int, [_int, _int, _int, _int, _P(CsrT)]),
    "spmm_c_bsr_stats_from_csr_host": (_int, [_P(CsrT), _P(BsrStatsT)]),
    "spmm_c_bsr_from_csr_device": (_int, [_P(CsrT), _P(BsrT), _vp]),
    "spmm_c_bsr_stats_from_csr_device": (_int, [_P(CsrT), _P(BsrStatsT), _vp]),
    "spmm_c_bsr_to_host": (_int, [_P(BsrT), _P(BsrT)]),
    "spmm_c_gpu_count": (_int, []),
    "spmm_c_unified": (_int, [_P(CsrT), _vp, _vp, _int, _int, _int, _P(_float), _P(_int)]),
    "spmm_c_generate_power_law_csr": (_int, [_int, _int, _double, _double, _int, _int, _P(CsrT)]),
    "spmm_c_round_to_fp16": (_int, [_vp, _long]),
    "spmm_c_nnz_balanced_bounds": (_int, [_P(CsrT), _int, _vp]),
    "spmm_c_compare": (_int, [_vp, _vp, _long, _P(_float), _P(_float), _P(_float)]),
    "spmm_c_host_reference_f64": (_int, [_P(CsrT), _vp, _int, _int, _vp]),
    "spmm_c_host_reference_bsr_f32": (_int, [_P(BsrT), _vp, _int, _int, _vp]),
    "spmm_c_baseline": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_memopt": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_memopt_v2": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_tiled": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_tiled_v2": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_tiled_v3": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_tiled_v4": (_int, [_P(CsrT), _vp, _vp, _int, _vp]),
    "spmm_c_tiled_v3_partitioned": (_int, [_P(CsrT), _vp, _int, _vp, _vp, _int, _vp]),
    "spmm_c_nnz_split_rows": (_int, [_P(CsrT), _int, _vp]),
    "spmm_c_split_partition_parts": (_int, [_int]),
    "spmm_c_tiled_v3_split": (_int, [_P(CsrT), _vp, _int, _vp, _vp, _int, _vp, _vp]),
    "spmm_c_tiled_v3_split_noalloc": (_int, [_P(CsrT), _vp, _int, _vp, _vp, _int, _vp]),
    "spmm_c_launch_repeat_split": (_int, [_P(CsrT), _vp, _int, _vp, _vp, _int, _vp, _int, _vp]),
    "spmm_c_default_partition_parts": (_int, [_int, _int]),
    "spmm_c_khalf_plan_create": (_int, [_P(CsrT), _int, _P(_vp)]),
    "spmm_c_khalf_launch": (_int, [_vp, _vp, _vp, _vp]),
    "spmm_c_khalf_plan_destroy": (None, [_vp]),
    "spmm_c_khalf_runs": (_int, [_vp, _int, ctypes.c_longlong, _vp, _int, _vp, _vp]),
    "spmm_c_launch_repeat_khalf": (_int, [_vp, _vp, _vp, _int, _vp]),
    "spmm_c_csr_auto_form": (_int, [_P(CsrT), _int, _P(ctypes.c_int),
                                    _P(EngineOptsT), _P(ctypes.c_int)]),
    "spmm_c_tiled_v3_opts": (_int, [_P(CsrT), _vp, _vp, _int, _P(EngineOptsT), _vp]),
    "spmm_c_float_to_half": (_int, [_vp, _vp, _long, _vp]),
    "spmm_c_wmma": (_int, [_P(BsrT), _vp, _vp, _int, _vp]),
    "spmm_c_wmma_opts": (_int, [_P(BsrT), _vp, _vp, _int, _P(BsrOptsT), _vp]),
    "spmm_c_launch_repeat_wmma_opts": (_int, [_P(BsrT), _vp, _vp, _int, _P(BsrOptsT), _int, _vp]),
    "spmm_c_bsr_tile_plan_create": (_int, [_P(BsrT), _int, _vp, _P(_vp)]),
    "spmm_c_bsr_tile_launch": (_int, [_vp, _P(BsrT), _vp, _vp, _int, _int, _vp]),
    "spmm_c_bsr_tile_plan_destroy": (None, [_vp]),
    "spmm_c_bsr_tile_plan_info": (_int, [_vp, _P(ctypes.c_int), _P(ctypes.c_int),
                                         _P(ctypes.c_int)]),
    "spmm_c_bsr_tile_records": (_int, [_vp, _vp, _int, _int, _int, _vp, _P(ctypes.c_int)]),
    "spmm_c_bsr_tile_shape_count": (_int, []),
    "spmm_c_bsr_tile_shape": (_int, [_int, _vp]),
    "spmm_c_bsr_tile_default_shape": (_int, [_vp, _int]),
    "spmm_c_launch_repeat_bsr_tile": (_int, [_vp, _P(BsrT), _vp, _vp, _int, _int, _int, _vp]),
    "spmm_c_hybrid_default_threshold": (_float, []),
    "spmm_c_hybrid_default_threshold_for": (_float, [ctypes.c_int]),
    "spmm_c_hybrid_choose": (_int, [_P(CsrT), _int, _float, _P(HybridPlanT)]),
    "spmm_c_backend_name": (ctypes.c_char_p, [_int]),
    "spmm_c_hybrid_run": (_int, [_P(HybridPlanT), _P(CsrT), _vp, _vp, _int, _int, _int, _P(_float)]),
    "spmm_c_launch_repeat": (_int, [_int, _vp, _vp, _vp, _int, _int, _vp]),
    "spmm_c_launch_repeat_opts": (_int, [_P(CsrT), _vp, _vp, _int, _P(EngineOptsT), _int, _vp]),
    "spmm_c_time_repeat": (_int, [_int, _vp, _vp, _vp, _int, _int, _vp, _P(_float)]),
    "spmm_c_device_synchronize": (_int, []),
    "spmm_c_shader_clock_trace": (_int, [_vp, _int, _int, _vp]),
}

_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return LIB_PATH


def _adopt_torch_hip_runtime() -> None:
    """Make the process hold exactly one HIP runtime.

    torch bundles its own libamdhip64 (SONAME libamdhip64.so.7) and loads it by
    a different file name than the system one.  If libspmm_amd.so is loaded
    first, the system runtime comes in with it and torch later brings a second
    copy; the two cannot share the device (launches then fail with "no
    ROCm-capable device").  Importing torch first makes the dynamic loader
    resolve the engine's libamdhip64.so.7 dependency to torch's copy.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib() -> ctypes.CDLL:
    """Load libspmm_amd.so (built by ``make -C sparse-matrix-multiplication_amd``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SpmmError(SPMM_INVALID, f"{LIB_PATH} is not built; run "
                            "`make -C sparse-matrix-multiplication_amd` (or __graft_entry__.build())")
        _adopt_torch_hip_runtime()
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _check(rc: int) -> None:
    if rc != SPMM_OK:
        raise SpmmError(rc, lib().spmm_c_last_error().decode())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data if a.size else 0


# ---------------------------------------------------------------------------
# Host CSR / BSR (copies out of the library's malloc'd arrays)
# ---------------------------------------------------------------------------
@dataclass
class HostCSR:
    """Host CSR (spmm::CSR, reference csr.h:7-14) held as numpy arrays."""
    num_rows: int
    num_cols: int
    row_ptr: np.ndarray  # int32[num_rows + 1]
    col_idx: np.ndarray  # int32[nnz]
    values: np.ndarray   # float32[nnz]

    @property
    def nnz(self) -> int:
        return int(self.col_idx.size)

    def struct(self) -> CsrT:
        self.row_ptr = np.ascontiguousarray(self.row_ptr, dtype=np.int32)
        self.col_idx = np.ascontiguousarray(self.col_idx, dtype=np.int32)
        self.values = np.ascontiguousarray(self.values, dtype=np.float32)
        return CsrT(self.num_rows, self.num_cols, self.nnz, _ptr(self.row_ptr),
                    _ptr(self.col_idx), _ptr(self.values))

    def to_dense(self) -> np.ndarray:
        d = np.zeros((self.num_rows, self.num_cols), dtype=np.float64)
        rows = np.repeat(np.arange(self.num_rows), np.diff(self.row_ptr))
        np.add.at(d, (rows, self.col_idx), self.values.astype(np.float64))
        return d


@dataclass
class HostBSR:
    """Host BSR (spmm::BSR_host, reference bsr.h:25-42); values are fp16 bits."""
    num_rows: int
    num_cols: int
    block_rows: int
    block_cols: int
    nnz: int
    row_ptr: np.ndarray   # int32[block_rows + 1]
    col_idx: np.ndarray   # int32[num_blocks]
    values: np.ndarray    # uint16[num_blocks * 256]

    @property
    def num_blocks(self) -> int:
        return int(self.col_idx.size)

    def struct(self) -> BsrT:
        self.row_ptr = np.ascontiguousarray(self.row_ptr, dtype=np.int32)
        self.col_idx = np.ascontiguousarray(self.col_idx, dtype=np.int32)
        self.values = np.ascontiguousarray(self.values, dtype=np.uint16)
        return BsrT(self.num_rows, self.num_cols, self.block_rows, self.block_cols,
                    self.num_blocks, self.nnz, _ptr(self.row_ptr), _ptr(self.col_idx),
                    _ptr(self.values))


def _csr_from_struct(s: CsrT) -> HostCSR:
    """Copy a library-owned host CSR into numpy and free the library copy."""
    try:
        rp = np.ctypeslib.as_array(ctypes.cast(s.row_ptr, _P(ctypes.c_int32)),
                                   (s.num_rows + 1,)).copy()
        ci = (np.ctypeslib.as_array(ctypes.cast(s.col_idx, _P(ctypes.c_int32)), (s.nnz,)).copy()
              if s.nnz else np.zeros(0, np.int32))
        va = (np.ctypeslib.as_array(ctypes.cast(s.values, _P(ctypes.c_float)), (s.nnz,)).copy()
              if s.nnz else np.zeros(0, np.float32))
        return HostCSR(s.num_rows, s.num_cols, rp, ci, va)
    finally:
        lib().spmm_c_csr_free_host(ctypes.byref(s))


def _bsr_from_struct(s: BsrT) -> HostBSR:
    try:
        rp = np.ctypeslib.as_array(ctypes.cast(s.row_ptr, _P(ctypes.c_int32)),
                                   (s.block_rows + 1,)).copy()
        ci = (np.ctypeslib.as_array(ctypes.cast(s.col_idx, _P(ctypes.c_int32)),
                                    (s.num_blocks,)).copy()
              if s.num_blocks else np.zeros(0, np.int32))
        va = (np.ctypeslib.as_array(ctypes.cast(s.values, _P(ctypes.c_uint16)),
                                    (s.num_blocks * 256,)).copy()
              if s.num_blocks else np.zeros(0, np.uint16))
        return HostBSR(s.num_rows, s.num_cols, s.block_rows, s.block_cols, s.nnz, rp, ci, va)
    finally:
        lib().spmm_c_bsr_free_host(ctypes.byref(s))


def generate_uniform_random_csr(rows: int, cols: int, density: float, seed: int) -> HostCSR:
    """Reference csr.cu:74-103."""
    s = CsrT()
    _check(lib().spmm_c_generate_uniform_random_csr(rows, cols, density, seed, ctypes.byref(s)))
    return _csr_from_struct(s)


def generate_banded_csr(rows: int, cols: int, half_bandwidth: int, seed: int) -> HostCSR:
    s = CsrT()
    _check(lib().spmm_c_generate_banded_csr(rows, cols, half_bandwidth, seed, ctypes.byref(s)))
    return _csr_from_struct(s)


def generate_block_diagonal_csr(rows: int, cols: int, block: int, seed: int,
                                value_scale: float = 0.1) -> HostCSR:
    s = CsrT()
    _check(lib().spmm_c_generate_block_diagonal_csr(rows, cols, block, seed, value_scale,
                                                    ctypes.byref(s)))
    return _csr_from_struct(s)


def generate_block_diagonal_uniform_csr(rows: int, cols: int, block: int, seed: int) -> HostCSR:
    """Block-diagonal structure with U[-1,1) values (gen_matrices.py:51-63)."""
    s = CsrT()
    _check(lib().spmm_c_generate_block_diagonal_uniform_csr(rows, cols, block, seed,
                                                            ctypes.byref(s)))
    return _csr_from_struct(s)


def generate_power_law_csr(rows: int, cols: int, mean_deg: float, alpha: float,
                           max_row_nnz: int, seed: int) -> HostCSR:
    s = CsrT()
    _check(lib().spmm_c_generate_power_law_csr(rows, cols, mean_deg, alpha, max_row_nnz, seed,
                                               ctypes.byref(s)))
    return _csr_from_struct(s)


def generate_dense_row_major(rows: int, cols: int, seed: int) -> np.ndarray:
    """Reference harness.cu:114-120."""
    out = np.empty((rows, cols), dtype=np.float32)
    _check(lib().spmm_c_generate_dense_row_major(rows, cols, seed, _ptr(out)))
    return out


def round_to_fp16(a: np.ndarray) -> np.ndarray:
    out = np.ascontiguousarray(a, dtype=np.float32).copy()
    _check(lib().spmm_c_round_to_fp16(_ptr(out), out.size))
    return out


def csr_from_coo_host(rows: int, cols: int, r, c, v) -> HostCSR:
    """Reference csr.cu:44-72."""
    r = np.ascontiguousarray(r, dtype=np.int32)
    c = np.ascontiguousarray(c, dtype=np.int32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    if not (r.size == c.size == v.size):
        raise SpmmError(SPMM_INVALID, "csr_from_coo_host: triplet size mismatch")
    n = int(v.size)
    s = CsrT()
    _check(lib().spmm_c_csr_from_coo_host(rows, cols, n, _ptr(r), _ptr(c), _ptr(v),
                                          ctypes.byref(s)))
    return _csr_from_struct(s)


def csr_row_slice_host(m: HostCSR, row_begin: int, row_end: int) -> HostCSR:
    s = CsrT()
    src = m.struct()
    _check(lib().spmm_c_csr_row_slice_host(ctypes.byref(src), row_begin, row_end, ctypes.byref(s)))
    return _csr_from_struct(s)


def csr_read_binary_host(path: str) -> HostCSR:
    s = CsrT()
    _check(lib().spmm_c_csr_read_binary_host(os.fsencode(path), ctypes.byref(s)))
    return _csr_from_struct(s)


def csr_write_binary_host(m: HostCSR, path: str) -> None:
    src = m.struct()
    _check(lib().spmm_c_csr_write_binary_host(ctypes.byref(src), os.fsencode(path)))


def bsr_from_csr_host(m: HostCSR) -> HostBSR:
    """Reference bsr.cu:30-109."""
    s = BsrT()
    src = m.struct()
    _check(lib().spmm_c_bsr_from_csr_host(ctypes.byref(src), ctypes.byref(s)))
    return _bsr_from_struct(s)


def bsr_compute_stats(b: HostBSR) -> BsrStatsT:
    st = BsrStatsT()
    src = b.struct()
    _check(lib().spmm_c_bsr_compute_stats(ctypes.byref(src), ctypes.byref(st)))
    return st


def bsr_stats_from_csr_host(m: HostCSR) -> BsrStatsT:
    """bsr_compute_stats(bsr_from_csr_host(m)) without building the blocks."""
    st = BsrStatsT()
    src = m.struct()
    _check(lib().spmm_c_bsr_stats_from_csr_host(ctypes.byref(src), ctypes.byref(st)))
    return st


def nnz_balanced_bounds(m: HostCSR, parts: int) -> np.ndarray:
    out = np.empty(parts + 1, dtype=np.int32)
    src = m.struct()
    _check(lib().spmm_c_nnz_balanced_bounds(ctypes.byref(src), parts, _ptr(out)))
    return out


def default_partition_parts(num_rows: int, nnz: int) -> int:
    return int(lib().spmm_c_default_partition_parts(num_rows, nnz))


def nnz_split_rows(m: HostCSR, parts: int) -> np.ndarray:
    """Row table of the merge-path partition (parts + 1 ints)."""
    out = np.empty(parts + 1, dtype=np.int32)
    src = m.struct()
    _check(lib().spmm_c_nnz_split_rows(ctypes.byref(src), parts, _ptr(out)))
    return out


def split_partition_parts(nnz: int) -> int:
    return int(lib().spmm_c_split_partition_parts(nnz))


_CSR_FORMS = {0: "engine", 1: "rowgroups", 2: "split", 3: "khalf"}


def csr_auto_form(m: HostCSR, N: int):
    """The CSR form spmm_hybrid_run picks: (name, EngineOptsT, merge-path parts)."""
    src = m.struct()
    form, parts = ctypes.c_int(), ctypes.c_int()
    opts = EngineOptsT()
    _check(lib().spmm_c_csr_auto_form(ctypes.byref(src), N, ctypes.byref(form), ctypes.byref(opts),
                                      ctypes.byref(parts)))
    return _CSR_FORMS[form.value], opts, parts.value


def compare(ours: np.ndarray, ref: np.ndarray):
    """Reference harness.cu:179-196 -> (max_abs, max_rel, rel_l2)."""
    a = np.ascontiguousarray(ours, dtype=np.float32).ravel()
    b = np.ascontiguousarray(ref, dtype=np.float32).ravel()
    ma, mr, rl = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
    _check(lib().spmm_c_compare(_ptr(a), _ptr(b), a.size, ctypes.byref(ma), ctypes.byref(mr),
                                ctypes.byref(rl)))
    return ma.value, mr.value, rl.value


def host_reference_f64(m: HostCSR, B: np.ndarray, threads: int = 0) -> np.ndarray:
    B = np.ascontiguousarray(B, dtype=np.float32)
    N = B.shape[1]
    out = np.empty((m.num_rows, N), dtype=np.float32)
    src = m.struct()
    _check(lib().spmm_c_host_reference_f64(ctypes.byref(src), _ptr(B), N, threads, _ptr(out)))
    return out


@dataclass
class Plan:
    backend: int
    fill_in_ratio: float
    block_density: float
    threshold: float
    n_aligned: bool
    reason: str

    @property
    def backend_name(self) -> str:
        return lib().spmm_c_backend_name(self.backend).decode()


def hybrid_default_threshold(N: Optional[int] = None) -> float:
    """The MI355X fill-in cut-off for a B of N columns (the wide-B value when
    N is not given)."""
    if N is None:
        return float(lib().spmm_c_hybrid_default_threshold())
    return float(lib().spmm_c_hybrid_default_threshold_for(int(N)))


def hybrid_choose(m: HostCSR, N: int, threshold: Optional[float] = None) -> Plan:
    """Reference spmm_hybrid.cu:32-56."""
    if threshold is None:
        threshold = -1.0  # the per-N MI355X crossover
    p = HybridPlanT()
    src = m.struct()
    _check(lib().spmm_c_hybrid_choose(ctypes.byref(src), N, threshold, ctypes.byref(p)))
    return Plan(p.backend, p.fill_in_ratio, p.block_density, p.threshold, bool(p.n_aligned),
                p.reason.decode())


def backend_name(backend: int) -> str:
    return lib().spmm_c_backend_name(backend).decode()


def gpu_count() -> int:
    """Reference spmm_multigpu.h:32."""
    return int(lib().spmm_c_gpu_count())


def _host_b(m: HostCSR, B) -> np.ndarray:
    """Host B as a contiguous float32 K x N array with K = A's columns (the C++
    side copies K * N floats from it)."""
    B = np.ascontiguousarray(B, dtype=np.float32)
    if B.ndim != 2 or B.shape[0] != m.num_cols:
        raise SpmmError(SPMM_INVALID, f"B: shape {B.shape}, expected ({m.num_cols}, N)")
    return B


def unified_run(m: HostCSR, B: np.ndarray, warmup: int = 3, iters: int = 10):
    """Reference spmm_unified (spmm_multigpu.cu:122-182): host in, host out ->
    (C, median ms, residency): 1 managed and prefetched, 0 managed but moved on
    first touch, -1 no managed memory on the device (device copies instead)."""
    B = _host_b(m, B)
    N = B.shape[1]
    C = np.empty((m.num_rows, N), dtype=np.float32)
    ms = ctypes.c_float()
    moved = ctypes.c_int()
    src = m.struct()
    _check(lib().spmm_c_unified(ctypes.byref(src), _ptr(B), _ptr(C), N, warmup, iters,
                                ctypes.byref(ms), ctypes.byref(moved)))
    return C, ms.value, moved.value


def hybrid_run(plan: Plan, m: HostCSR, B: np.ndarray, warmup: int = 3, iters: int = 10):
    """Reference spmm_hybrid.cu:58-125: host in, host out -> (C, median ms)."""
    B = _host_b(m, B)
    N = B.shape[1]
    C = np.empty((m.num_rows, N), dtype=np.float32)
    p = HybridPlanT(plan.backend, plan.fill_in_ratio, plan.block_density, plan.threshold,
                    int(plan.n_aligned), plan.reason.encode())
    ms = ctypes.c_float()
    src = m.struct()
    _check(lib().spmm_c_hybrid_run(ctypes.byref(p), ctypes.byref(src), _ptr(B), _ptr(C), N,
                                   warmup, iters, ctypes.byref(ms)))
    return C, ms.value


# ---------------------------------------------------------------------------
# Device side (torch tensors as HBM buffers)
# ---------------------------------------------------------------------------
def _torch():
    import torch  # imported lazily: host-only users never need it
    return torch


def _stream_handle(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)



def _device_of(A):
    """The device holding a DeviceCSR / DeviceBSR's arrays (None for a library-built BSR)."""
    rp = getattr(A, "row_ptr", None)
    return rp.device if rp is not None and hasattr(rp, "device") else None


def _check_dense(t, name: str, dtypes, rows: Optional[int] = None, cols: Optional[int] = None,
                 device=None, ndim: int = 2):
    """Validate a device operand before any launch: a contiguous cuda tensor of
    one of `dtypes` with the expected shape.  The C ABI takes bare pointers and
    sizes, so a wrong tensor here would otherwise read or write out of bounds
    on the device; raises SpmmError(SPMM_INVALID) instead."""
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise SpmmError(SPMM_INVALID, f"{name}: expected a torch tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise SpmmError(SPMM_INVALID, f"{name}: must be a cuda tensor (got {t.device})")
    if device is not None and t.device != device:
        raise SpmmError(SPMM_INVALID, f"{name}: on {t.device}, the matrix is on {device}")
    if t.dtype not in dtypes:
        want = " or ".join(str(d) for d in dtypes)
        raise SpmmError(SPMM_INVALID, f"{name}: dtype {t.dtype}, expected {want}")
    if not t.is_contiguous():
        raise SpmmError(SPMM_INVALID, f"{name}: must be contiguous (row-major)")
    if t.dim() != ndim:
        raise SpmmError(SPMM_INVALID, f"{name}: expected {ndim}-D, got shape {tuple(t.shape)}")
    if rows is not None and int(t.shape[0]) != rows:
        raise SpmmError(SPMM_INVALID, f"{name}: {int(t.shape[0])} rows, expected {rows}")
    if cols is not None and ndim == 2 and int(t.shape[1]) != cols:
        raise SpmmError(SPMM_INVALID, f"{name}: {int(t.shape[1])} columns, expected {cols}")


def _csr_operands(A, B, C, fp16: bool = False):
    """Check B (K x N) and C (M x N, float32; allocated when None) against A;
    returns (N, C).  fp16: B holds fp16 values (float16, or int16 bit patterns)."""
    torch = _torch()
    dev = _device_of(A)
    bt = (torch.float16, torch.int16) if fp16 else (torch.float32,)
    _check_dense(B, "B", bt, rows=A.num_cols, device=dev)
    N = int(B.shape[1])
    if C is None:
        C = torch.empty((A.num_rows, N), dtype=torch.float32, device=B.device)
    else:
        _check_dense(C, "C", (torch.float32,), rows=A.num_rows, cols=N, device=B.device)
    return N, C


class DeviceCSR:
    """Device CSR whose three arrays are torch tensors (spmm::CSR with HBM pointers)."""

    def __init__(self, host: HostCSR, device: str = "cuda"):
        torch = _torch()
        self.num_rows, self.num_cols, self.nnz = host.num_rows, host.num_cols, host.nnz
        self.row_ptr = torch.from_numpy(np.ascontiguousarray(host.row_ptr, np.int32)).to(device)
        self.col_idx = torch.from_numpy(np.ascontiguousarray(host.col_idx, np.int32)).to(device)
        self.values = torch.from_numpy(np.ascontiguousarray(host.values, np.float32)).to(device)

    def struct(self) -> CsrT:
        return CsrT(self.num_rows, self.num_cols, self.nnz, self.row_ptr.data_ptr(),
                    self.col_idx.data_ptr() if self.nnz else 0,
                    self.values.data_ptr() if self.nnz else 0)


class DeviceBSR:
    """Device BSR (spmm::BSR): fp16 blocks as an int16 torch tensor of bit patterns."""

    def __init__(self, host: HostBSR, device: str = "cuda"):
        torch = _torch()
        self.num_rows, self.num_cols = host.num_rows, host.num_cols
        self.block_rows, self.block_cols = host.block_rows, host.block_cols
        self.num_blocks, self.nnz = host.num_blocks, host.nnz
        self.row_ptr = torch.from_numpy(np.ascontiguousarray(host.row_ptr, np.int32)).to(device)
        self.col_idx = torch.from_numpy(np.ascontiguousarray(host.col_idx, np.int32)).to(device)
        self.values = torch.from_numpy(
            np.ascontiguousarray(host.values, np.uint16).view(np.int16)).to(device)

    def struct(self) -> BsrT:
        return BsrT(self.num_rows, self.num_cols, self.block_rows, self.block_cols,
                    self.num_blocks, self.nnz, self.row_ptr.data_ptr(),
                    self.col_idx.data_ptr() if self.num_blocks else 0,
                    self.values.data_ptr() if self.num_blocks else 0)


class BuiltDeviceBSR:
    """A device BSR whose arrays the library allocated (bsr_from_csr_device);
    released with spmm_c_bsr_free_device when the object goes away."""

    def __init__(self, s: BsrT):
        self._s = s
        self.num_rows, self.num_cols = s.num_rows, s.num_cols
        self.block_rows, self.block_cols = s.block_rows, s.block_cols
        self.num_blocks, self.nnz = s.num_blocks, s.nnz

    def struct(self) -> BsrT:
        return self._s

    def to_host(self) -> HostBSR:
        h = BsrT()
        _check(lib().spmm_c_bsr_to_host(ctypes.byref(self._s), ctypes.byref(h)))
        return _bsr_from_struct(h)

    def free(self) -> None:
        if self._s is not None:
            lib().spmm_c_bsr_free_device(ctypes.byref(self._s))
            self._s = None

    def __del__(self):
        try:
            self.free()
        except Exception:  # interpreter shutdown
            pass


def bsr_from_csr_device(A: DeviceCSR, stream=None) -> BuiltDeviceBSR:
    """CSR -> BSR on the device (same arrays as bsr_from_csr_host)."""
    s = BsrT()
    src = A.struct()
    _check(lib().spmm_c_bsr_from_csr_device(ctypes.byref(src), ctypes.byref(s),
                                            _stream_handle(stream)))
    return BuiltDeviceBSR(s)


def bsr_stats_from_csr_device(A: DeviceCSR, stream=None) -> BsrStatsT:
    st = BsrStatsT()
    src = A.struct()
    _check(lib().spmm_c_bsr_stats_from_csr_device(ctypes.byref(src), ctypes.byref(st),
                                                  _stream_handle(stream)))
    return st


def spmm_csr(kernel: str, A: DeviceCSR, B, C=None, stream=None):
    """Launch one of the seven CSR entry points (reference src/kernels/spmm_*.h).

    B: cuda float32 tensor (K x N), C: optional cuda float32 (M x N) output."""
    torch = _torch()
    if kernel not in CSR_KERNELS:
        raise SpmmError(SPMM_INVALID, f"unknown CSR kernel {kernel!r}")
    N, C = _csr_operands(A, B, C)
    s = A.struct()
    fn = getattr(lib(), f"spmm_c_{kernel}")
    _check(fn(ctypes.byref(s), B.data_ptr(), C.data_ptr(), N, _stream_handle(stream)))
    return C


def spmm_tiled_v3_partitioned(A: DeviceCSR, bounds, B, C=None, stream=None):
    torch = _torch()
    N, C = _csr_operands(A, B, C)
    _check_dense(bounds, "bounds", (torch.int32,), device=B.device, ndim=1)
    if bounds.numel() < 2:
        raise SpmmError(SPMM_INVALID, "bounds: needs parts + 1 >= 2 entries")
    s = A.struct()
    _check(lib().spmm_c_tiled_v3_partitioned(ctypes.byref(s), bounds.data_ptr(),
                                             int(bounds.numel()) - 1, B.data_ptr(),
                                             C.data_ptr(), N, _stream_handle(stream)))
    return C


def spmm_tiled_v3_split(A: DeviceCSR, split_rows, B, C=None, carry=None, stream=None):
    """Merge-path partition: split_rows = cuda int32 tensor of parts+1 rows."""
    torch = _torch()
    N, C = _csr_operands(A, B, C)
    parts = _check_split(split_rows, B, N, carry)
    if carry is None:
        carry = torch.empty((max(parts, 1), max(N, 1)), dtype=torch.float32, device=B.device)
    s = A.struct()
    _check(lib().spmm_c_tiled_v3_split(ctypes.byref(s), split_rows.data_ptr(), parts,
                                       B.data_ptr(), C.data_ptr(), N, carry.data_ptr(),
                                       _stream_handle(stream)))
    return C


def _check_split(split_rows, B, N: int, carry) -> int:
    """Check the merge-path row table and carry workspace; returns parts."""
    torch = _torch()
    _check_dense(split_rows, "split_rows", (torch.int32,), device=B.device, ndim=1)
    parts = int(split_rows.numel()) - 1
    if parts < 1:
        raise SpmmError(SPMM_INVALID, "split_rows: needs parts + 1 >= 2 entries")
    if carry is not None:
        _check_dense(carry, "carry", (torch.float32,), device=B.device, ndim=carry.dim())
        if carry.numel() < parts * N:
            raise SpmmError(SPMM_INVALID, f"carry: {carry.numel()} floats, needs parts * N = "
                                          f"{parts * N}")
    return parts


def spmm_tiled_v3_split_noalloc(A: DeviceCSR, split_rows, B, C=None, stream=None):
    """Merge-path partition with the carries in the library's per-GPU device
    array (allocates nothing; parts x N <= 2**19; overlapping calls on one GPU
    race)."""
    N, C = _csr_operands(A, B, C)
    parts = _check_split(split_rows, B, N, None)
    s = A.struct()
    _check(lib().spmm_c_tiled_v3_split_noalloc(ctypes.byref(s), split_rows.data_ptr(), parts,
                                               B.data_ptr(), C.data_ptr(), N,
                                               _stream_handle(stream)))
    return C


class KHalfPlan:
    """Merge-path launch over B-row halves (no counterpart in the reference; the
    CSR form "khalf" spmm_hybrid_run picks when B is over one XCD's 4 MiB L2 at
    full width and half of its rows fit).  Built once from a host CSR for B of
    N columns; owns its device copies of the two halves and its workspaces
    (release with close(), or use it as a context manager).  Launches of one
    plan share those workspaces and must not overlap."""

    def __init__(self, A: "HostCSR", N: int):
        _torch()  # the HIP runtime comes in through torch first
        self.num_rows, self.num_cols, self.N = A.num_rows, A.num_cols, int(N)
        handle = ctypes.c_void_p()
        src = A.struct()
        _check(lib().spmm_c_khalf_plan_create(ctypes.byref(src), self.N, ctypes.byref(handle)))
        self._h = handle

    def _operands(self, B, C):
        torch = _torch()
        _check_dense(B, "B", (torch.float32,), rows=self.num_cols, cols=self.N)
        if C is None:
            C = torch.empty((self.num_rows, self.N), dtype=torch.float32, device=B.device)
        else:
            _check_dense(C, "C", (torch.float32,), rows=self.num_rows, cols=self.N,
                         device=B.device)
        if self._h is None:
            raise SpmmError(SPMM_INVALID, "plan is closed")
        return C

    def launch(self, B, C=None, stream=None):
        C = self._operands(B, C)
        _check(lib().spmm_c_khalf_launch(self._h, B.data_ptr(), C.data_ptr(),
                                         _stream_handle(stream)))
        return C

    def launch_repeat(self, B, C, reps: int, stream=None) -> None:
        """reps back-to-back launches (measurement helper)."""
        C = self._operands(B, C)
        _check(lib().spmm_c_launch_repeat_khalf(self._h, B.data_ptr(), C.data_ptr(), reps,
                                                _stream_handle(stream)))

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            lib().spmm_c_khalf_plan_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


TILE_SHAPE_FIELDS = ("R", "NT", "WC", "CS", "NB", "KIND")


def bsr_tile_shapes():
    """The run-panel kernel's shapes: a list of dicts with TILE_SHAPE_FIELDS."""
    out = []
    for i in range(lib().spmm_c_bsr_tile_shape_count()):
        f = np.zeros(6, np.int32)
        _check(lib().spmm_c_bsr_tile_shape(i, _ptr(f)))
        out.append(dict(zip(TILE_SHAPE_FIELDS, (int(x) for x in f))))
    return out


def bsr_tile_records(row_ptr, col_idx, block_cols: int, rows_per_panel: int = 4):
    """Host part of the run-panel plan: (records (panels x 32 int32), widest
    union).  Raises SpmmError(SPMM_UNSUPPORTED) unless every block-row is a
    run of consecutive block-columns and each panel's runs cover their union."""
    rp = np.ascontiguousarray(row_ptr, np.int32)
    ci = np.ascontiguousarray(col_idx, np.int32)
    block_rows = rp.size - 1
    panels = (block_rows + rows_per_panel - 1) // rows_per_panel
    rec = np.zeros((max(panels, 1), 32), np.int32)
    mu = ctypes.c_int()
    _check(lib().spmm_c_bsr_tile_records(_ptr(rp), _ptr(ci) if ci.size else 0, block_rows,
                                         int(block_cols), int(rows_per_panel), _ptr(rec),
                                         ctypes.byref(mu)))
    return rec[:panels], mu.value


class BsrTilePlan:
    """Run-panel plan of a device BSR (no counterpart in the reference; the
    form of spmm_wmma that spmm_hybrid_run runs on structured matrices).  One
    record per panel of rows_per_panel block-rows; creation reads the BSR's
    block structure back from the device.  Raises SpmmError(SPMM_UNSUPPORTED)
    when the structure is not runs (use launch_repeat("wmma", ...) then)."""

    def __init__(self, A, rows_per_panel: int = 4, stream=None):
        _torch()
        self.A = A
        self.num_rows, self.num_cols = A.num_rows, A.num_cols
        self._h = None
        handle = ctypes.c_void_p()
        s = A.struct()
        _check(lib().spmm_c_bsr_tile_plan_create(ctypes.byref(s), int(rows_per_panel),
                                                 _stream_handle(stream), ctypes.byref(handle)))
        self._h = handle
        panels, rpp, mu = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(lib().spmm_c_bsr_tile_plan_info(self._h, ctypes.byref(panels), ctypes.byref(rpp),
                                               ctypes.byref(mu)))
        self.panels, self.rows_per_panel, self.max_union = panels.value, rpp.value, mu.value

    def default_shape(self, N: int) -> int:
        return int(lib().spmm_c_bsr_tile_default_shape(self._h, int(N)))

    def _operands(self, B16, C):
        if self._h is None:
            raise SpmmError(SPMM_INVALID, "plan is closed")
        return _csr_operands(self.A, B16, C, fp16=True)

    def launch(self, B16, C=None, shape: int = -1, stream=None):
        N, C = self._operands(B16, C)
        s = self.A.struct()
        _check(lib().spmm_c_bsr_tile_launch(self._h, ctypes.byref(s), B16.data_ptr(),
                                            C.data_ptr(), N, int(shape), _stream_handle(stream)))
        return C

    def launch_repeat(self, B16, C, reps: int, shape: int = -1, stream=None) -> None:
        """reps back-to-back launches (measurement helper)."""
        N, C = self._operands(B16, C)
        s = self.A.struct()
        _check(lib().spmm_c_launch_repeat_bsr_tile(self._h, ctypes.byref(s), B16.data_ptr(),
                                                   C.data_ptr(), N, int(shape), int(reps),
                                                   _stream_handle(stream)))

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            lib().spmm_c_bsr_tile_plan_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def khalf_runs(row_ptr, nnz: int, split_rows):
    """Host helper of the B-row halves fix-up: per row, the first and last
    merge-path part continuing it (-1 when none) -> (first, last) int32 arrays."""
    rp = np.ascontiguousarray(row_ptr, np.int32)
    rows = np.ascontiguousarray(split_rows, np.int32)
    M = rp.size - 1
    first = np.empty(max(M, 0), np.int32)
    last = np.empty(max(M, 0), np.int32)
    _check(lib().spmm_c_khalf_runs(_ptr(rp), M, int(nnz), _ptr(rows), rows.size - 1,
                                   _ptr(first), _ptr(last)))
    return first, last


def launch_repeat_split(A: DeviceCSR, split_rows, B, C, carry, reps: int, stream=None) -> None:
    """reps back-to-back merge-path launches (measurement helper)."""
    N, C = _csr_operands(A, B, C)
    _check_split(split_rows, B, N, carry)
    if carry is None:
        raise SpmmError(SPMM_INVALID, "carry: a workspace of parts * N floats is required")
    s = A.struct()
    _check(lib().spmm_c_launch_repeat_split(ctypes.byref(s), split_rows.data_ptr(),
                                            int(split_rows.numel()) - 1, B.data_ptr(),
                                            C.data_ptr(), int(B.shape[1]), carry.data_ptr(),
                                            reps, _stream_handle(stream)))


def spmm_tiled_v3_opts(A: DeviceCSR, B, opts: EngineOptsT, C=None, stream=None):
    N, C = _csr_operands(A, B, C)
    s = A.struct()
    _check(lib().spmm_c_tiled_v3_opts(ctypes.byref(s), B.data_ptr(), C.data_ptr(), N,
                                      ctypes.byref(opts), _stream_handle(stream)))
    return C


def shader_clock_trace(samples: int, interval_us: float, stream=None):
    """Starts a shader-clock trace on `stream` (spmm_c_shader_clock_trace):
    one wave samples shader cycles and 100 MHz real-time ticks `samples`
    times, `interval_us` apart.  Returns the device buffer for
    shader_clock_series; launch it on a second stream beside a workload."""
    torch = _torch()
    out = torch.zeros(2 * samples, dtype=torch.int64, device="cuda")
    _check(lib().spmm_c_shader_clock_trace(out.data_ptr(), samples,
                                           max(1, int(round(interval_us * 100))),
                                           _stream_handle(stream)))
    return out


def shader_clock_series(out) -> list:
    """[(t_us from the first sample, MHz over the interval ending there)] of a
    finished shader_clock_trace buffer."""
    v = out.cpu().numpy().reshape(-1, 2).astype(np.float64)
    c, r = v[:, 0], v[:, 1]
    return [(float((r[i] - r[0]) / 100.0), float(100.0 * (c[i] - c[i - 1]) / (r[i] - r[i - 1])))
            for i in range(1, len(v)) if r[i] > r[i - 1]]


def shader_clock_mhz(interval_us: float = 10.0, stream=None) -> float:
    """The shader clock delivered now (one 10 us interval, synchronised)."""
    torch = _torch()
    out = shader_clock_trace(2, interval_us, stream)
    torch.cuda.synchronize()
    return shader_clock_series(out)[-1][1]


def float_to_half(src, dst=None, stream=None):
    """Reference spmm_wmma.cu:125-130: fp32 -> fp16 (RNE) on the device."""
    torch = _torch()
    _check_dense(src, "src", (torch.float32,), ndim=src.dim() if hasattr(src, "dim") else 1)
    if dst is None:
        dst = torch.empty(src.shape, dtype=torch.float16, device=src.device)
    else:
        _check_dense(dst, "dst", (torch.float16, torch.int16), device=src.device, ndim=dst.dim())
        if dst.numel() != src.numel():
            raise SpmmError(SPMM_INVALID, f"dst: {dst.numel()} elements, src has {src.numel()}")
    _check(lib().spmm_c_float_to_half(src.data_ptr(), dst.data_ptr(), src.numel(),
                                      _stream_handle(stream)))
    return dst


def spmm_wmma(A: DeviceBSR, B16, C=None, stream=None):
    """Reference spmm_wmma.cu:132-142: BSR x fp16 B -> fp32 C on matrix cores."""
    N, C = _csr_operands(A, B16, C, fp16=True)
    s = A.struct()
    _check(lib().spmm_c_wmma(ctypes.byref(s), B16.data_ptr(), C.data_ptr(), N,
                             _stream_handle(stream)))
    return C


def spmm_wmma_opts(A: DeviceBSR, B16, opts: BsrOptsT, C=None, stream=None):
    """spmm_wmma with explicit kernel options (row group, column tiles, per-wave)."""
    N, C = _csr_operands(A, B16, C, fp16=True)
    s = A.struct()
    _check(lib().spmm_c_wmma_opts(ctypes.byref(s), B16.data_ptr(), C.data_ptr(), N,
                                  ctypes.byref(opts), _stream_handle(stream)))
    return C


def launch_repeat_wmma_opts(A: DeviceBSR, B16, C, opts: BsrOptsT, reps: int, stream=None) -> None:
    N, C = _csr_operands(A, B16, C, fp16=True)
    s = A.struct()
    _check(lib().spmm_c_launch_repeat_wmma_opts(ctypes.byref(s), B16.data_ptr(), C.data_ptr(),
                                                int(B16.shape[1]), ctypes.byref(opts), reps,
                                                _stream_handle(stream)))


def launch_repeat(kernel: str, A, B, C, reps: int, stream=None) -> None:
    if kernel not in KERNEL_IDS:
        raise SpmmError(SPMM_INVALID, f"unknown kernel {kernel!r}")
    N, C = _csr_operands(A, B, C, fp16=(kernel == "wmma"))
    s = A.struct()
    _check(lib().spmm_c_launch_repeat(KERNEL_IDS[kernel], ctypes.byref(s), B.data_ptr(),
                                      C.data_ptr(), int(B.shape[1]), reps, _stream_handle(stream)))


def launch_repeat_opts(A: DeviceCSR, B, C, opts: EngineOptsT, reps: int, stream=None) -> None:
    N, C = _csr_operands(A, B, C)
    s = A.struct()
    _check(lib().spmm_c_launch_repeat_opts(ctypes.byref(s), B.data_ptr(), C.data_ptr(),
                                           int(B.shape[1]), ctypes.byref(opts), reps,
                                           _stream_handle(stream)))


def time_repeat(kernel: str, A, B, C, reps: int, stream=None) -> float:
    """Milliseconds for `reps` back-to-back launches between two hipEvents on `stream`."""
    if kernel not in KERNEL_IDS:
        raise SpmmError(SPMM_INVALID, f"unknown kernel {kernel!r}")
    N, C = _csr_operands(A, B, C, fp16=(kernel == "wmma"))
    s = A.struct()
    ms = ctypes.c_float()
    _check(lib().spmm_c_time_repeat(KERNEL_IDS[kernel], ctypes.byref(s), B.data_ptr(),
                                    C.data_ptr(), int(B.shape[1]), reps, _stream_handle(stream),
                                    ctypes.byref(ms)))
    return ms.value
