"""The generator CLI (role of scripts/gen_matrices.py) and the pattern-sweep
driver's parsing (role of scripts/run_pattern_sweep.py), on the CPU."""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                   "sparse-matrix-multiplication_amd")


def _gen(tmp_path, *args):
    out = str(tmp_path / "m.bin")
    env = dict(os.environ, PYTHONPATH=PKG)
    r = subprocess.run([sys.executable, "-m", "spmm_amd.gen_matrices", *args, "--out", out],
                       env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return out, r.stdout.strip()


def _read_raw(path):
    """The binary CSR layout written by csr_write_binary_host (csr.cu:125-150)."""
    data = open(path, "rb").read()
    rows, cols, nnz = struct.unpack("<iii", data[:12])
    off = 12
    rp = np.frombuffer(data, "<i4", rows + 1, off); off += 4 * (rows + 1)
    ci = np.frombuffer(data, "<i4", nnz, off); off += 4 * nnz
    va = np.frombuffer(data, "<f4", nnz, off); off += 4 * nnz
    assert off == len(data)
    return rows, cols, rp, ci, va


def test_uniform_known_answer(S, tmp_path):
    # generate_uniform_random_csr(1024, 1024, 0.01, 42) has 10388 nonzeros
    # (the reference's committed sweep, reports/data/sweep.csv)
    path, line = _gen(tmp_path, "--pattern", "uniform", "--rows", "1024", "--cols", "1024")
    rows, cols, rp, ci, va = _read_raw(path)
    assert (rows, cols, rp[-1]) == (1024, 1024, 10388)
    assert line == f"wrote {path}  rows=1024 cols=1024 nnz=10388 density={10388 / 1024**2:.6f}"
    A = S.csr_read_binary_host(path)
    ref = S.generate_uniform_random_csr(1024, 1024, 0.01, 42)
    assert np.array_equal(A.col_idx, ref.col_idx) and np.array_equal(A.values, ref.values)


def test_banded_default_bandwidth(tmp_path):
    path, _ = _gen(tmp_path, "--pattern", "banded", "--rows", "100", "--cols", "80")
    rows, cols, rp, ci, va = _read_raw(path)
    # default half-bandwidth 16: row r holds columns max(0, r-16) .. min(80, r+17) - 1
    want = [min(80, r + 17) - max(0, r - 16) if r - 16 < 80 else 0 for r in range(100)]
    assert list(np.diff(rp)) == want
    for r in (0, 20, 95):
        cols_r = ci[rp[r]:rp[r + 1]]
        assert np.array_equal(cols_r, np.arange(max(0, r - 16), min(80, r + 17)))
    assert np.all((va >= -1) & (va < 1))


def test_block_diagonal_default_block(S, tmp_path):
    path, _ = _gen(tmp_path, "--pattern", "block-diagonal", "--rows", "100", "--cols", "130",
                   "--seed", "5")
    rows, cols, rp, ci, va = _read_raw(path)
    # default block 32: floor(100 / 32) = 3 dense blocks, rows 96..99 empty
    assert rp[-1] == 3 * 32 * 32
    assert list(np.diff(rp)) == [32] * 96 + [0] * 4
    assert np.array_equal(ci[rp[40]:rp[41]], np.arange(32, 64))
    # values: U[-1,1) in CSR order, the dense generator's stream of the same seed
    assert np.array_equal(va, S.generate_dense_row_major(1, rp[-1], 5).ravel())


def test_power_law_defaults(tmp_path):
    path, _ = _gen(tmp_path, "--pattern", "power-law", "--rows", "4000", "--cols", "500")
    rows, cols, rp, ci, va = _read_raw(path)
    deg = np.diff(rp)
    assert deg.min() >= 1 and deg.max() <= 500          # clipped to [1, cols]
    assert abs(deg.mean() - 16.0) < 1.0                  # default mean-deg 16
    for r in range(0, 4000, 397):
        row = ci[rp[r]:rp[r + 1]]
        assert np.all(np.diff(row) > 0)                  # distinct, sorted


def test_unknown_pattern_rejected(tmp_path):
    env = dict(os.environ, PYTHONPATH=PKG)
    r = subprocess.run([sys.executable, "-m", "spmm_amd.gen_matrices", "--pattern", "bogus",
                        "--rows", "4", "--cols", "4", "--out", str(tmp_path / "x.bin")],
                       env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "invalid choice" in r.stderr


def test_parse_kernel_lines():
    sys.path.insert(0, PKG)
    from spmm_amd.run_pattern_sweep import parse_kernel_lines
    out = ("bsr_stats blocks=4 stored_elems=1024\n"
           "kernel=tiled_v3 m=64 k=64 n=128 nnz=410 density=0.100098 time_ms=0.0051 "
           "gflops=20.50 max_abs_err=1.1e-06 rel_l2_err=1.0e-07 single_ms=0.0079 hbm_gbs=9.1 "
           "pct_hbm=0.11 cold_ms=0.0123 cpu_ms=0.101 cpu_threads=8 cpu_gflops=1.0\n"
           "kernel=hybrid[wmma] m=64 k=64 n=128 nnz=410 density=0.1 time_ms=0.01 gflops=10.0\n"
           "kernel=broken m=64 time_ms=\n")
    recs = list(parse_kernel_lines(out))
    assert [r["kernel"] for r in recs] == ["tiled_v3", "hybrid[wmma]"]
    assert recs[0]["m"] == 64 and recs[0]["nnz"] == 410 and recs[0]["cpu_threads"] == 8
    assert recs[0]["cold_ms"] == pytest.approx(0.0123)
