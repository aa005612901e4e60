"""The engine's host side (C++ API through the C ABI, no GPU needed) against
the oracle and the reference's documented behaviour: generators, COO->CSR,
binary format, row slices, BSR build and statistics, dispatch, partition and
metrics, and the error conditions the reference raises."""
import os
import struct

import numpy as np
import pytest


def test_uniform_generator_bitwise_equals_oracle(S, O):
    for (m, k, d, seed) in ((1024, 1024, 0.01, 42), (300, 700, 0.05, 9), (64, 1, 0.5, 3)):
        A = S.generate_uniform_random_csr(m, k, d, seed)
        rp, ci, va = O.uniform_csr(m, k, d, seed)
        assert np.array_equal(A.row_ptr, rp)
        assert np.array_equal(A.col_idx, ci)
        assert np.array_equal(A.values.view(np.uint32), va.view(np.uint32))


@pytest.mark.parametrize("m,d,nnz", [(4096, 0.01, 167686), (8192, 0.01, 671114),
                                     (4096, 0.05, 839236)])
def test_uniform_generator_known_nnz(S, m, d, nnz):
    assert S.generate_uniform_random_csr(m, m, d, 42).nnz == nnz


def test_uniform_generator_rejects_bad_density(S):
    for d in (-0.1, 1.5, float("nan")):
        with pytest.raises(S.SpmmError) as e:
            S.generate_uniform_random_csr(10, 10, d, 1)
        assert "invalid density" in str(e.value)
    assert S.generate_uniform_random_csr(5, 7, 1.0, 1).nnz == 35
    assert S.generate_uniform_random_csr(5, 7, 0.0, 1).nnz == 0


def test_dense_generator_bitwise_equals_oracle(S, O):
    a = S.generate_dense_row_major(129, 77, 43)
    assert np.array_equal(a.view(np.uint32), O.dense(129, 77, 43).view(np.uint32))


def test_coo_to_csr_matches_oracle(S, O):
    rng = np.random.default_rng(8)
    n = 4000
    r = rng.integers(0, 150, n)
    c = rng.integers(0, 90, n)
    r[:100], c[:100] = r[100:200], c[100:200]
    v = rng.standard_normal(n).astype(np.float32)
    A = S.csr_from_coo_host(150, 90, r, c, v)
    rp, ci, va = O.coo_to_csr(150, r, c, v)
    assert np.array_equal(A.row_ptr, rp) and np.array_equal(A.col_idx, ci)
    assert np.array_equal(A.values, va) and A.nnz == n


def test_coo_errors(S):
    with pytest.raises(S.SpmmError):
        S.csr_from_coo_host(3, 3, [0, 1], [0], [1.0, 2.0])
    with pytest.raises(S.SpmmError):
        S.csr_from_coo_host(3, 3, [0, 3], [0, 0], [1.0, 2.0])  # row out of range


def test_binary_format_round_trip_and_layout(S, tmp_path):
    A = S.generate_uniform_random_csr(50, 60, 0.1, 5)
    path = str(tmp_path / "a.bin")
    S.csr_write_binary_host(A, path)
    raw = open(path, "rb").read()
    hdr = struct.unpack("<iii", raw[:12])
    assert hdr == (50, 60, A.nnz)
    assert len(raw) == 12 + 4 * 51 + 8 * A.nnz
    body = np.frombuffer(raw[12:], dtype=np.uint8)
    assert np.array_equal(body[:4 * 51].view("<i4"), A.row_ptr)
    assert np.array_equal(body[4 * 51:4 * 51 + 4 * A.nnz].view("<i4"), A.col_idx)
    assert np.array_equal(body[4 * 51 + 4 * A.nnz:].view("<f4"), A.values)
    B = S.csr_read_binary_host(path)
    assert np.array_equal(B.row_ptr, A.row_ptr) and np.array_equal(B.col_idx, A.col_idx)
    assert np.array_equal(B.values, A.values) and (B.num_rows, B.num_cols) == (50, 60)


def test_binary_format_errors(S, tmp_path):
    with pytest.raises(S.SpmmError) as e:
        S.csr_read_binary_host(str(tmp_path / "missing.bin"))
    assert e.value.code == S.SPMM_IO_ERROR and "cannot open" in str(e.value)
    short = tmp_path / "short.bin"
    short.write_bytes(struct.pack("<ii", 1, 2))
    with pytest.raises(S.SpmmError) as e:
        S.csr_read_binary_host(str(short))
    assert "short read on header" in str(e.value)
    body = tmp_path / "body.bin"
    body.write_bytes(struct.pack("<iii", 4, 4, 10) + b"\0" * 8)
    with pytest.raises(S.SpmmError) as e:
        S.csr_read_binary_host(str(body))
    assert "short read on body" in str(e.value)


def test_row_slice(S):
    A = S.generate_uniform_random_csr(40, 30, 0.2, 2)
    s = S.csr_row_slice_host(A, 10, 25)
    assert s.num_rows == 15 and s.num_cols == 30
    assert s.row_ptr[0] == 0 and s.nnz == A.row_ptr[25] - A.row_ptr[10]
    assert np.array_equal(s.to_dense(), A.to_dense()[10:25])
    assert S.csr_row_slice_host(A, 5, 5).nnz == 0
    for bad in ((-1, 3), (3, 41), (20, 10)):
        with pytest.raises(S.SpmmError) as e:
            S.csr_row_slice_host(A, *bad)
        assert "invalid row range" in str(e.value)


def test_bsr_build_equals_oracle(S, O):
    rng = np.random.default_rng(12)
    for (M, K) in ((1024, 1024), (45, 70), (17, 300)):
        A = S.generate_uniform_random_csr(M, K, 0.03, int(rng.integers(1000)))
        b = S.bsr_from_csr_host(A)
        brp, bci, bv = O.bsr_build(M, K, A.row_ptr, A.col_idx, A.values)
        assert np.array_equal(b.row_ptr, brp) and np.array_equal(b.col_idx, bci)
        assert np.array_equal(b.values, bv)
        assert (b.block_rows, b.block_cols) == ((M + 15) // 16, (K + 15) // 16)


def test_bsr_duplicates_keep_last(S, O):
    A = S.csr_from_coo_host(20, 20, [3, 3, 3], [4, 4, 9], [1.0, 2.0, 3.0])
    b = S.bsr_from_csr_host(A)
    blk = b.values.view(np.float16).reshape(-1, 16, 16)[0].astype(np.float32)
    assert blk[3, 4] == 2.0 and blk[3, 9] == 3.0


@pytest.mark.parametrize("m,d,known", [(4096, 0.01, (60630, 15521280, 92.6, 0.925)),
                                       (1024, 0.05, (4096, 1048576, 20.1, 1.0))])
def test_bsr_stats_known_answers(S, m, d, known):
    st = S.bsr_compute_stats(S.bsr_from_csr_host(S.generate_uniform_random_csr(m, m, d, 42)))
    assert (st.num_blocks, st.stored_elements) == known[:2]
    assert round(st.fill_in_ratio, 1) == known[2] and round(st.block_density, 3) == known[3]


def test_config_patterns(S):
    b = S.generate_banded_csr(8192, 8192, 64, 1003)
    assert b.nnz == 1052608
    st = S.bsr_compute_stats(S.bsr_from_csr_host(b))
    assert st.num_blocks == 4588 and round(st.fill_in_ratio, 4) == 1.1158
    rows = np.repeat(np.arange(8192), np.diff(b.row_ptr))
    assert np.all(np.abs(rows - b.col_idx) <= 64)
    d = S.generate_block_diagonal_csr(8192, 8192, 256, 2003, 0.1)
    assert d.nnz == 32 * 256 * 256
    st = S.bsr_compute_stats(S.bsr_from_csr_host(d))
    assert st.num_blocks == 8192 and st.fill_in_ratio == 1.0
    assert np.all(d.col_idx // 256 == np.repeat(np.arange(8192), 256) // 256)
    assert abs(float(d.values.std()) - 0.1) < 0.002 and abs(float(d.values.mean())) < 0.002
    p = S.generate_power_law_csr(16384, 16384, 164.0, 1.5, 4096, 3003)
    deg = np.diff(p.row_ptr)
    assert deg.max() == 4096 and deg.min() >= 1
    assert 0.008 < p.nnz / 16384**2 < 0.011
    for r in (0, int(np.argmax(deg)), 16383):
        row = p.col_idx[p.row_ptr[r]:p.row_ptr[r + 1]]
        assert np.all(np.diff(row) > 0)  # distinct, sorted
    # power-law tail: a heavy top percentile
    top = np.sort(deg)[-164:].sum() / p.nnz
    assert top > 0.1


def test_power_law_small_distribution(S):
    # Pareto x_m = 1, alpha: P(x > t) = t^-alpha before scaling; degree ratios
    # to the minimum follow the same tail
    p = S.generate_power_law_csr(200000, 100000, 20.0, 2.5, 100000, 11)
    deg = np.diff(p.row_ptr).astype(np.float64)
    x = deg / deg.min()
    for t in (2.0, 4.0):
        frac = float(np.mean(x > t))
        assert abs(frac - t ** -2.5) < 0.02, (t, frac)


def test_round_to_fp16(S):
    x = np.array([1.0, 1.0004883, 65520.0, 1e-8, -2.5], np.float32)
    with np.errstate(over="ignore"):  # 65520 rounds to inf in fp16
        want = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(S.round_to_fp16(x), want)


def test_hybrid_choose_matches_oracle_rule(S, O):
    A = S.generate_banded_csr(256, 256, 3, 1)
    fill = S.bsr_compute_stats(S.bsr_from_csr_host(A)).fill_in_ratio
    reasons = {0: "low BSR fill-in and N aligned to 16 -> Tensor Cores",
               1: "N not a multiple of 16 -> CUDA-core CSR",
               2: "high BSR fill-in -> CUDA-core CSR"}
    for N in (0, 8, 16, 17, 128):
        for thr in (1.0, fill, 2.0, 6.0):
            p = S.hybrid_choose(A, N, thr)
            use, why = O.hybrid_rule(fill, N, thr)
            assert p.backend == use and p.reason == reasons[why], (N, thr)
            assert p.n_aligned == (N > 0 and N % 16 == 0)
            assert p.fill_in_ratio == pytest.approx(fill)
    assert S.backend_name(0) == "csr" and S.backend_name(1) == "wmma"
    # the MI355X crossover by width of B: 8 (N <= 16) .. 32 (N >= 256); this
    # matrix has fill ~6.6 -> matrix cores at every N, and an explicit
    # threshold keeps the reference's rule
    assert S.hybrid_default_threshold() == 32.0
    for N, thr in ((16, 8.0), (32, 12.0), (48, 16.0), (64, 16.0), (128, 24.0), (256, 32.0),
                   (1024, 32.0)):
        assert S.hybrid_default_threshold(N) == thr
        p = S.hybrid_choose(A, N)
        assert p.threshold == thr and p.backend_name == "wmma"
    p = S.hybrid_choose(A, 128, 5.0)
    assert p.threshold == 5.0 and p.backend_name == "csr"


def test_nnz_balanced_bounds_equals_oracle(S, O):
    A = S.generate_power_law_csr(3000, 3000, 30.0, 1.5, 1000, 4)
    for parts in (1, 2, 7, 256, 4000):
        assert np.array_equal(S.nnz_balanced_bounds(A, parts), O.nnz_balanced_bounds(A.row_ptr, parts))
    with pytest.raises(S.SpmmError):
        S.nnz_balanced_bounds(A, 0)
    assert 256 <= S.default_partition_parts(16384, 2_500_000) <= 16384
    assert S.default_partition_parts(10, 100) == 10


def test_compare_equals_oracle(S, O):
    rng = np.random.default_rng(2)
    a = rng.standard_normal(5000).astype(np.float32)
    b = a + rng.standard_normal(5000).astype(np.float32) * 1e-3
    assert np.allclose(S.compare(a, b), O.compare(a, b), rtol=1e-6)


def test_host_reference_equals_oracle(S, O):
    A = S.generate_power_law_csr(500, 800, 30.0, 1.5, 400, 6)
    B = S.generate_dense_row_major(800, 48, 7)
    C64, _ = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=2)
    for threads in (1, 3):
        C = S.host_reference_f64(A, B, threads)
        assert np.array_equal(C, C64.astype(np.float32))


def test_bsr_stats_from_csr_host_equals_full_build(S):
    cases = [S.generate_uniform_random_csr(300, 500, 0.03, 1),
             S.generate_banded_csr(1000, 1000, 37, 3),
             S.generate_power_law_csr(3000, 2500, 40.0, 1.5, 2500, 5),
             S.csr_from_coo_host(48, 128, [0, 0, 5, 17, 17], [3, 3, 9, 100, 2],
                                 [1.0, 2.0, 3.0, 4.0, 5.0]),
             S.csr_from_coo_host(77, 33, [], [], [])]
    for A in cases:
        fast = S.bsr_stats_from_csr_host(A)
        full = S.bsr_compute_stats(S.bsr_from_csr_host(A))
        for f in ("num_blocks", "stored_elements", "original_nnz", "fill_in_ratio",
                  "block_density"):
            assert getattr(fast, f) == getattr(full, f), f


def test_csr_auto_form(S):
    # the CSR form spmm_hybrid_run picks from the row lengths (host only):
    # row groups, the engine with the longest row as hint, or merge-path
    c1 = S.generate_uniform_random_csr(4096, 4096, 0.01, 42)
    c2 = S.generate_uniform_random_csr(8192, 8192, 0.01, 42)
    c5 = S.generate_power_law_csr(16384, 16384, 164.0, 1.5, 4096, 3003)
    longest = lambda m: int(np.diff(m.row_ptr).max())
    form, opts, parts = S.csr_auto_form(c1, 128)  # >= 4096 even rows at N = 128
    assert (form, opts.row_groups, opts.max_row_hint, parts) == ("rowgroups", 1, longest(c1), 0)
    form, opts, parts = S.csr_auto_form(c2, 128)  # 8192 rows of 82: the engine's one round
    assert (form, opts.row_groups, opts.max_row_hint, parts) == ("engine", 0, longest(c2), 0)
    # a 4096-entry row: merge-path; B of 8 MiB (over one XCD's 4 MiB L2, half of
    # it within): over B-row halves, which choose their own parts
    form, opts, parts = S.csr_auto_form(c5, 128)
    assert (form, parts) == ("khalf", 0)
    assert longest(c5) == 4096
    assert S.csr_auto_form(c5, 120)[0] == "khalf"   # 7.5 MiB, N % 4 == 0
    assert S.csr_auto_form(c5, 130)[0] == "split"   # N % 4 != 0
    assert S.csr_auto_form(c5, 256)[0] == "split"   # half of B is 8 MiB
    # a long row, but only 100 entries in the upper half of the columns (a
    # half needs 512): plain merge-path
    rows = np.r_[np.repeat(np.arange(16384), 12), np.zeros(3000, np.int64)]
    cols = np.r_[(np.arange(16384 * 12) * 7919) % 8192, np.arange(3000) * 2]
    cols[:100] += 8192
    lop = S.csr_from_coo_host(16384, 16384, rows, cols, np.ones(rows.size, np.float32))
    assert longest(lop) > 2560
    assert S.csr_auto_form(lop, 128)[0] == "split"
    assert S.csr_auto_form(c2, 16)[0] == "rowgroups"
    assert S.csr_auto_form(c2, 256)[0] == "engine"
    # N = 16: four column lanes take rows up to 16384 / 4 = 4096 entries
    assert S.csr_auto_form(c5, 16)[0] == "rowgroups"
    # N = 64: 16 column lanes, rows up to 1024 (or 8x the average) -> merge-path
    assert S.csr_auto_form(c5, 64)[0] == "split"
    # power-law rows capped at 512 pass the skew test but are not even: the engine
    pl = S.generate_power_law_csr(16384, 16384, 164.0, 1.5, 512, 5)
    assert longest(pl) <= 512
    assert S.csr_auto_form(pl, 128)[0] == "engine"
    assert S.csr_auto_form(pl, 16)[0] == "rowgroups"
    # no nonzeros: the engine, no hint
    empty = S.csr_from_coo_host(8, 8, [], [], [])
    assert S.csr_auto_form(empty, 32)[:2][0] == "engine"
    with pytest.raises(S.SpmmError) as e:
        S.csr_auto_form(c1, -1)
    assert e.value.code == S.SPMM_INVALID


def test_nnz_split_rows_definition(S):
    # rows[g] = last row r < M with row_ptr[r] <= nnz*g/parts; rows[0] = 0, rows[parts] = M
    rng = np.random.default_rng(12)
    mats = [S.generate_power_law_csr(500, 400, 20.0, 1.5, 400, 3),
            S.csr_from_coo_host(50, 30, [3, 3, 3, 40, 41, 41], [0, 5, 9, 1, 2, 3], np.ones(6)),
            S.csr_from_coo_host(20, 2000, np.full(1500, 7), rng.permutation(2000)[:1500],
                                rng.uniform(-1, 1, 1500))]
    for A in mats:
        for parts in (1, 2, 3, 7, 64, A.nnz, A.nnz + 5):
            rows = S.nnz_split_rows(A, parts)
            assert rows[0] == 0 and rows[parts] == A.num_rows
            assert np.all(np.diff(rows) >= 0)
            for g in range(1, parts):
                p = A.nnz * g // parts
                want = max(r for r in range(A.num_rows) if A.row_ptr[r] <= p)
                assert rows[g] == want, (g, p)
                assert A.row_ptr[rows[g]] <= p < A.row_ptr[rows[g] + 1]  # the row holds p
    with pytest.raises(S.SpmmError):
        S.nnz_split_rows(S.csr_from_coo_host(4, 4, [], [], []), 3)


def test_khalf_runs(S):
    # Per row, the merge-path parts that continue it (their piece of the row
    # goes to the carry the B-row halves' fix-up adds).  Checked against a
    # restatement over entries: part g continues a row exactly when its first
    # entry and the entry before it belong to the same row.
    for seed, (M, parts) in enumerate([(2000, 64), (300, 512), (50, 7), (1, 3)]):
        A = S.generate_power_law_csr(M, M * 4, 40.0, 1.5, 1500, seed + 11)
        if A.nnz < parts:
            continue
        rows = S.nnz_split_rows(A, parts)
        first, last = S.khalf_runs(A.row_ptr, A.nnz, rows)
        row_of = np.repeat(np.arange(M), np.diff(A.row_ptr))
        want_first = np.full(M, -1)
        want_last = np.full(M, -1)
        for g in range(parts):
            lo, hi = A.nnz * g // parts, A.nnz * (g + 1) // parts
            if lo < hi and lo > 0 and row_of[lo] == row_of[lo - 1]:
                r = row_of[lo]
                if want_first[r] < 0:
                    want_first[r] = g
                want_last[r] = g
        assert np.array_equal(first, want_first) and np.array_equal(last, want_last)
        # a run is a block of consecutive parts, all inside the row
        for r in np.nonzero(first >= 0)[0]:
            for g in range(first[r], last[r] + 1):
                assert row_of[A.nnz * g // parts] == r
    # a row split over many parts: one long row in the middle
    A = S.csr_from_coo_host(3, 100, [0] * 5 + [1] * 90 + [2] * 5, list(range(5)) + list(range(90)) +
                            list(range(5)), np.ones(100, np.float32))
    first, last = S.khalf_runs(A.row_ptr, A.nnz, S.nnz_split_rows(A, 10))
    assert first.tolist() == [-1, 1, -1] and last.tolist() == [-1, 9, -1]


def test_khalf_runs_errors(S):
    import ctypes
    rp = np.array([0, 2, 4], np.int32)
    rows = np.array([0, 2], np.int32)
    first = np.empty(2, np.int32)
    last = np.empty(2, np.int32)
    L = S.lib()
    # parts < 1, negative sizes, missing arrays
    assert L.spmm_c_khalf_runs(S._ptr(rp), 2, 4, S._ptr(rows), 0, S._ptr(first),
                               S._ptr(last)) == S.SPMM_INVALID
    assert L.spmm_c_khalf_runs(S._ptr(rp), -1, 4, S._ptr(rows), 1, S._ptr(first),
                               S._ptr(last)) == S.SPMM_INVALID
    assert L.spmm_c_khalf_runs(None, 2, 4, S._ptr(rows), 1, S._ptr(first),
                               S._ptr(last)) == S.SPMM_INVALID
    assert L.spmm_c_khalf_runs(S._ptr(rp), 2, 4, None, 1, S._ptr(first),
                               S._ptr(last)) == S.SPMM_INVALID
    assert b"null" in L.spmm_c_last_error()
    # one part: nothing continues
    f, l = S.khalf_runs(rp, 4, rows)
    assert f.tolist() == [-1, -1] and l.tolist() == [-1, -1]
    # the plan entry points refuse null arguments without touching the GPU
    assert L.spmm_c_khalf_plan_create(None, 128, ctypes.byref(ctypes.c_void_p())) == \
        S.SPMM_INVALID
    assert L.spmm_c_khalf_launch(None, None, None, None) == S.SPMM_INVALID
    L.spmm_c_khalf_plan_destroy(None)
