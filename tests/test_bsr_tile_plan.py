"""Run-panel plan records (the host part of the plan build in bsr_tile.hip,
spmm_c_bsr_tile_records) on the CPU.

A record describes a panel of R block-rows: the union of their runs (first
block-column u0, width U) and per block-row its run as union slots [lo, hi)
and the A block of slot lo.  The checks are the invariants the kernel relies
on, restated from the BSR's own arrays: every slot of every run names the
block that holds that block-column (col_idx[ab + s - lo] == u0 + s), the runs
cover exactly the union, empty block-rows and panels have empty runs, and the
widest union is reported.  Structures that are not runs are refused.
"""
import numpy as np
import pytest

from spmm_amd import SPMM_UNSUPPORTED, SPMM_INVALID


def _check_records(hb, R, rec, max_union):
    rp, ci = np.asarray(hb.row_ptr), np.asarray(hb.col_idx)
    panels = (hb.block_rows + R - 1) // R
    assert rec.shape == (panels, 32)
    widest = 0
    for p in range(panels):
        u0, U = int(rec[p, 0]), int(rec[p, 1])
        covered = np.zeros(max(U, 0), bool)
        for r in range(R):
            br = p * R + r
            lo, hi, ab = (int(rec[p, 2 + r]), int(rec[p, 2 + R + r]), int(rec[p, 2 + 2 * R + r]))
            cnt = rp[br + 1] - rp[br] if br < hb.block_rows else 0
            assert hi - lo == cnt, (p, r)
            if cnt == 0:
                assert lo == hi == 0
                continue
            assert 0 <= lo < hi <= U
            assert ab == rp[br]
            for s in range(lo, hi):
                assert ci[ab + s - lo] == u0 + s, (p, r, s)
            covered[lo:hi] = True
        assert covered.all(), p  # no gap in the union
        if U == 0:
            assert u0 == 0
        widest = max(widest, U)
    assert max_union == widest


@pytest.mark.parametrize("R", [4, 8])
@pytest.mark.parametrize("kind,M,K,param", [
    ("band", 8192, 8192, 64),   # c3's structure
    ("band", 1000, 1000, 20),
    ("band", 300, 200, 0),      # diagonal only, ragged K
    ("band", 160, 160, 1),
    ("diag", 8192, 8192, 256),  # c4's structure
    ("diag", 1000, 1000, 40),   # diagonal blocks straddling block-rows
    ("diag", 512, 512, 512),
])
def test_records_structured(S, R, kind, M, K, param):
    A = (S.generate_banded_csr(M, K, param, 5) if kind == "band"
         else S.generate_block_diagonal_csr(M, K, param, 6, 0.1))
    hb = S.bsr_from_csr_host(A)
    rec, mu = S.bsr_tile_records(hb.row_ptr, hb.col_idx, hb.block_cols, R)
    _check_records(hb, R, rec, mu)


def test_records_known_answer(S):
    # five block-rows, runs 0-2, 1-3, 2-4, 3-5, 4-5 (a band), panels of four
    rp = np.array([0, 3, 6, 9, 12, 14], np.int32)
    ci = np.array([0, 1, 2, 1, 2, 3, 2, 3, 4, 3, 4, 5, 4, 5], np.int32)
    rec, mu = S.bsr_tile_records(rp, ci, 6, 4)
    assert mu == 6
    assert list(rec[0, :14]) == [0, 6, 0, 1, 2, 3, 3, 4, 5, 6, 0, 3, 6, 9]
    assert list(rec[1, :14]) == [4, 2, 0, 0, 0, 0, 2, 0, 0, 0, 12, 0, 0, 0]
    assert not rec[:, 14:].any()


def test_records_empty_rows_and_panels(S):
    # block-rows 0-3 empty (a zero panel), 4 and 6 hold runs, 5 and 7 empty
    rp = np.array([0, 0, 0, 0, 0, 2, 2, 5, 5], np.int32)
    ci = np.array([7, 8, 6, 7, 8], np.int32)
    rec, mu = S.bsr_tile_records(rp, ci, 10, 4)
    assert not rec[0].any()
    assert list(rec[1, :14]) == [6, 3, 1, 0, 0, 0, 3, 0, 3, 0, 0, 0, 2, 0]
    assert mu == 3


@pytest.mark.parametrize("rp,ci,why", [
    ([0, 2], [0, 2], "gap inside a row"),
    ([0, 2], [1, 0], "descending"),
    ([0, 2], [3, 3], "repeated block-column"),
    ([0, 1, 2], [0, 5], "runs of one panel leave a gap"),
    ([0, 1], [9], "block-column outside the matrix"),
])
def test_records_refused(S, rp, ci, why):
    with pytest.raises(S.SpmmError) as e:
        S.bsr_tile_records(np.array(rp, np.int32), np.array(ci, np.int32), 8, 4)
    assert e.value.code == SPMM_UNSUPPORTED, why


def test_records_bad_panel_rows(S):
    with pytest.raises(S.SpmmError) as e:
        S.bsr_tile_records(np.array([0, 1], np.int32), np.array([0], np.int32), 4, 3)
    assert e.value.code == SPMM_INVALID


def test_uniform_random_is_not_runs(S):
    hb = S.bsr_from_csr_host(S.generate_uniform_random_csr(512, 512, 0.01, 42))
    with pytest.raises(S.SpmmError) as e:
        S.bsr_tile_records(hb.row_ptr, hb.col_idx, hb.block_cols, 4)
    assert e.value.code == SPMM_UNSUPPORTED


def test_records_random_runs(S):
    # Seeded random run structures: the plan accepts exactly those whose panels'
    # runs cover their union without a gap (restated in tile_cases), and then
    # its records satisfy every invariant the kernel relies on.
    from tile_cases import random_case, panels_contiguous
    rng = np.random.default_rng(2024)
    accepted = refused = 0
    for case in range(120):
        A, runs, M, K = random_case(S, rng)
        hb = S.bsr_from_csr_host(A)
        assert list(np.diff(hb.row_ptr)) == [L for _, L in runs], case
        for R in (4, 8):
            if panels_contiguous(runs, R):
                rec, mu = S.bsr_tile_records(hb.row_ptr, hb.col_idx, hb.block_cols, R)
                _check_records(hb, R, rec, mu)
                accepted += 1
            else:
                with pytest.raises(S.SpmmError) as e:
                    S.bsr_tile_records(hb.row_ptr, hb.col_idx, hb.block_cols, R)
                assert e.value.code == SPMM_UNSUPPORTED, (case, R)
                refused += 1
    assert accepted >= 60 and refused >= 20, (accepted, refused)


def test_shapes_table(S):
    shapes = S.bsr_tile_shapes()
    assert shapes, "no kernel shapes"
    for sh in shapes:
        assert sh["R"] in (4, 8) and sh["KIND"] in (0, 1, 2, 3)
        assert sh["NT"] % 16 == 0 and sh["CS"] % 2 == 0 and 2 <= sh["NB"] <= 6
