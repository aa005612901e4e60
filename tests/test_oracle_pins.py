"""Pins of the CPU oracle against values the oracle does not compute itself:
the reference's committed known answers, independent library routines
(numpy's MT19937 and float16, scipy.sparse) and brute force.  Each test is
chosen so that a plausible slip in the restatement (wrong tempering constant,
FMA in the value draw, truncation instead of RNE, dropped duplicate, wrong
block offset) fails it.
"""
import numpy as np
import pytest
import scipy.sparse as sp

# (m = k, density) -> nnz of generate_uniform_random_csr(m, m, d, 42), from the
# reference's committed runs: reports/data/sweep.csv (nnz column) and
# scripts/roofline.py EMBEDDED.
KNOWN_NNZ = {
    (1024, 0.05): 52260, (1024, 0.01): 10388, (1024, 0.001): 1044,
    (4096, 0.05): 839236, (4096, 0.01): 167686, (4096, 0.001): 16935,
    (8192, 0.05): 3354625, (8192, 0.01): 671114, (8192, 0.001): 67137,
    (16384, 0.05): 13421456, (16384, 0.01): 2684748, (16384, 0.001): 268160,
}

# (m = k, density) -> (num_blocks, stored, fill (1 dp), block density (3 dp)),
# reports/tensor_core_wmma.md:43-56.
KNOWN_BSR = {
    (1024, 0.05): (4096, 1048576, 20.1, 1.000),
    (1024, 0.01): (3761, 962816, 92.7, 0.918),
    (1024, 0.001): (917, 234752, 224.9, 0.224),
    (4096, 0.05): (65536, 16777216, 20.0, 1.000),
    (4096, 0.01): (60630, 15521280, 92.6, 0.925),
    (4096, 0.001): (14924, 3820544, 225.6, 0.228),
    (8192, 0.01): (242248, 62015488, 92.4, 0.924),
    (8192, 0.001): (59324, 15186944, 226.2, 0.226),
}


def test_mt19937_matches_numpy_legacy_stream(O):
    for seed in (0, 1, 42, 43, 5489, 2**31 - 1):
        bg = np.random.MT19937()
        bg._legacy_seeding(seed)
        ref = bg.random_raw(3000).astype(np.uint32)
        assert np.array_equal(O.mt_raw(seed, 3000), ref), seed


def test_mt19937_standard_known_answer(O):
    # ISO C++ [rand.predef]: the 10000th invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995.
    assert int(O.mt_raw(5489, 10000)[-1]) == 4123659995


def test_canonical_float_rounding(O):
    # one 32-bit draw -> float(draw) / 2^32, pulled below 1.0 when it rounds up
    assert O.canonical_f32(0) == 0.0
    assert O.canonical_f32(1 << 31) == 0.5
    top = np.float32(np.nextafter(np.float32(1.0), np.float32(0.0)))
    assert O.canonical_f32(0xFFFFFFFF) == top          # rounds to 2^32 -> clamped
    assert O.canonical_f32(0xFFFFFF7F) == top          # largest draw below the tie
    assert O.canonical_f32(12345) == np.float32(12345) / np.float32(2**32)


@pytest.mark.parametrize("m,d", [(1024, 0.05), (1024, 0.01), (1024, 0.001),
                                 (4096, 0.05), (4096, 0.01), (4096, 0.001),
                                 (8192, 0.01)])
def test_uniform_generator_known_nnz(O, m, d):
    assert O.uniform_nnz(m, m, d, 42) == KNOWN_NNZ[(m, d)]


def test_uniform_generator_values_and_statistics(O):
    rp, ci, va = O.uniform_csr(2048, 1024, 0.03, 7)
    assert rp[0] == 0 and np.all(np.diff(rp) >= 0) and rp[-1] == ci.size
    for r in range(0, 2048, 97):
        row = ci[rp[r]:rp[r + 1]]
        assert np.all(np.diff(row) > 0)  # strictly ascending columns, no duplicates
    assert va.min() >= -1.0 and va.max() < 1.0
    assert abs(ci.size / (2048 * 1024) - 0.03) < 0.002
    assert abs(float(va.mean())) < 0.02


def test_dense_generator_is_the_value_stream(O):
    # B is one uniform(-1, 1) per element: value = canonical * 2 - 1 in float
    raw = O.mt_raw(43, 64)
    expect = (raw.astype(np.float32) / np.float32(2**32)) * np.float32(2.0) - np.float32(1.0)
    assert np.array_equal(O.dense(8, 8, 43).ravel().view(np.uint32), expect.view(np.uint32))


def test_coo_to_csr_matches_lexsort_with_duplicates(O):
    rng = np.random.default_rng(3)
    n, rows, cols = 5000, 300, 200
    r = rng.integers(0, rows, n).astype(np.int32)
    c = rng.integers(0, cols, n).astype(np.int32)
    r[:50] = r[50:100]  # force duplicate (row, col) pairs
    c[:50] = c[50:100]
    v = rng.standard_normal(n).astype(np.float32)
    rp, ci, va = O.coo_to_csr(rows, r, c, v)
    order = np.lexsort((c, r))  # stable: duplicates keep input order
    assert np.array_equal(ci, c[order])
    assert np.array_equal(va, v[order])
    assert np.array_equal(rp, np.concatenate([[0], np.cumsum(np.bincount(r, minlength=rows))]))
    assert ci.size == n  # nothing de-duplicated (csr.cu:44-72)


def test_coo_rejects_bad_row(O):
    with pytest.raises(ValueError):
        O.coo_to_csr(4, [0, 4], [0, 0], [1.0, 2.0])


def _scipy_ref(rp, ci, va, B):
    M = rp.size - 1
    A = sp.csr_matrix((va.astype(np.float64), ci, rp), shape=(M, B.shape[0]))
    return A @ B.astype(np.float64)


def test_csr_spmm_f64_matches_scipy(O):
    rp, ci, va = O.uniform_csr(700, 500, 0.02, 11)
    B = O.dense(500, 37, 12)
    for threads in (1, 4):
        C, absC = O.csr_spmm_f64(rp, ci, va, B, threads=threads)
        ref = _scipy_ref(rp, ci, va, B)
        assert np.allclose(C, ref, rtol=1e-13, atol=1e-13)
        absref = _scipy_ref(rp, ci, np.abs(va), np.abs(B))
        assert np.allclose(absC, absref, rtol=1e-13, atol=1e-13)


def test_csr_spmm_special_cases(O):
    B = O.dense(6, 5, 1)
    # identity -> C == B
    rp = np.arange(7, dtype=np.int32)
    ci = np.arange(6, dtype=np.int32)
    C, _ = O.csr_spmm_f64(rp, ci, np.ones(6, np.float32), B)
    assert np.array_equal(C, B.astype(np.float64))
    # empty rows -> zeros; single entry -> scaled row; duplicates are summed
    rp = np.array([0, 0, 1, 1, 3], np.int32)
    ci = np.array([4, 2, 2], np.int32)
    va = np.array([2.0, 0.5, 0.25], np.float32)
    C, _ = O.csr_spmm_f64(rp, ci, va, B)
    Bd = B.astype(np.float64)
    assert np.all(C[0] == 0) and np.all(C[2] == 0)
    assert np.array_equal(C[1], 2.0 * Bd[4])
    assert np.array_equal(C[3], 0.75 * Bd[2])  # both scalings are exact in fp64


def _fused_chain_f64(rp, ci, va, B):
    # Each step sum = fma(v, b, sum) restated in fp64: the product of two fp32
    # values is exact in fp64, the sum rounds once to fp64 and once to fp32
    # (equal to the single fused rounding unless the fp64 sum lands on an fp32
    # rounding midpoint, which these inputs never do).
    M, N = rp.size - 1, B.shape[1]
    C = np.zeros((M, N), np.float32)
    Bd = B.astype(np.float64)
    for r in range(M):
        s = np.zeros(N, np.float32)
        for p in range(rp[r], rp[r + 1]):
            s = (np.float64(va[p]) * Bd[ci[p]] + s.astype(np.float64)).astype(np.float32)
        C[r] = s
    return C


def test_csr_spmm_f32_fma_matches_a_step_restatement(O):
    rp, ci, va = O.uniform_csr(120, 90, 0.08, 21)
    B = O.dense(90, 13, 22)
    C = O.csr_spmm_f32_fma(rp, ci, va, B)
    assert np.array_equal(C.view(np.uint32), _fused_chain_f64(rp, ci, va, B).view(np.uint32))


def test_csr_spmm_f32_fma_exact_and_fused(O):
    # small integers: every product and partial sum is exact, so the chain is
    # the exact product
    rng = np.random.default_rng(5)
    rp = np.array([0, 3, 3, 7], np.int32)
    ci = rng.integers(0, 6, 7).astype(np.int32)
    va = rng.integers(-8, 9, 7).astype(np.float32)
    B = rng.integers(-50, 51, (6, 4)).astype(np.float32)
    C = O.csr_spmm_f32_fma(rp, ci, va, B)
    C64, _ = O.csr_spmm_f64(rp, ci, va, B)
    assert np.array_equal(C.astype(np.float64), C64) and np.all(C[1] == 0)
    # one fused step differs from multiply-then-add: after sum = -1, the
    # product (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 is exact inside the fused
    # operation (sum 2^-11 + 2^-24), while rounding it to fp32 first ties to
    # even at 1 + 2^-11 (sum 2^-11)
    x = np.float32(1 + 2.0 ** -12)
    rp = np.array([0, 2], np.int32)
    ci = np.array([0, 1], np.int32)
    va = np.array([1.0, x], np.float32)
    B = np.array([[-1.0], [x]], np.float32)
    C = O.csr_spmm_f32_fma(rp, ci, va, B)
    assert C[0, 0] == np.float32(2.0 ** -11 + 2.0 ** -24)
    assert np.float32(np.float32(x * x) + np.float32(-1.0)) == np.float32(2.0 ** -11)


def test_fp16_rne_matches_numpy(O):
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6,
                        6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08,
                        2.9802326e-08, 8.940697e-08, 1e-10, np.inf, -np.inf,
                        1.0009765625, 1.00048828125, 1.00146484375, 2049.0, 2051.0],
                       dtype=np.float32)
    # exact ties between fp16 neighbours: k + 0.5 ulp
    ties = (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0**-10) + np.float32(1.0)
            + np.float32(2.0**-11))
    rand = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s
                           for s in (1e-7, 1e-5, 1e-3, 1.0, 1e3, 6e4)])
    x = np.concatenate([special, ties, -ties, rand])
    got = O.f32_to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    back = np.array([O.f16_to_f32(int(h)) for h in got[:2000]], np.float32)
    assert np.array_equal(back, got[:2000].view(np.float16).astype(np.float32))
    nan = O.f32_to_f16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_fp16_to_f32_all_finite_patterns(O):
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(x)) for x in h[::7]], np.float32)
    assert np.array_equal(got, ref[::7])


def _dense_from_bsr(M, K, brp, bci, bv):
    out = np.zeros(((M + 15) // 16 * 16, (K + 15) // 16 * 16), np.float32)
    blocks = bv.view(np.float16).astype(np.float32).reshape(-1, 16, 16)
    for br in range(brp.size - 1):
        for b in range(brp[br], brp[br + 1]):
            out[br * 16:br * 16 + 16, bci[b] * 16:bci[b] * 16 + 16] = blocks[b]
    return out[:M, :K]


def test_bsr_build_brute_force(O):
    rng = np.random.default_rng(9)
    for M, K in ((50, 70), (16, 16), (33, 1), (1, 40)):
        n = max(1, M * K // 5)
        r = rng.integers(0, M, n)
        c = rng.integers(0, K, n)
        v = rng.standard_normal(n).astype(np.float32)
        rp, ci, va = O.coo_to_csr(M, r, c, v)
        brp, bci, bv = O.bsr_build(M, K, rp, ci, va)
        dense_last = np.zeros((M, K), np.float32)
        for i in range(rp.size - 1):  # the last duplicate in CSR order wins
            for p in range(rp[i], rp[i + 1]):
                dense_last[i, ci[p]] = va[p]
        assert np.array_equal(_dense_from_bsr(M, K, brp, bci, bv),
                              dense_last.astype(np.float16).astype(np.float32))
        # every stored block is non-empty in the source, columns ascending
        occupied = {(i // 16, ci[p] // 16) for i in range(M) for p in range(rp[i], rp[i + 1])}
        stored = {(br, bci[b]) for br in range(brp.size - 1) for b in range(brp[br], brp[br + 1])}
        assert occupied == stored
        for br in range(brp.size - 1):
            assert np.all(np.diff(bci[brp[br]:brp[br + 1]]) > 0)


@pytest.mark.parametrize("m,d", [(1024, 0.05), (1024, 0.01), (1024, 0.001),
                                 (4096, 0.01), (4096, 0.001)])
def test_bsr_known_answers(O, m, d):
    rp, ci, va = O.uniform_csr(m, m, d, 42)
    brp, bci, _ = O.bsr_build(m, m, rp, ci, va)
    nb = int(brp[-1])
    fill, dens, stored = O.bsr_stats(m, m, nb, ci.size)
    kb, ks, kf, kd = KNOWN_BSR[(m, d)]
    assert (nb, stored) == (kb, ks)
    assert round(fill, 1) == kf and round(dens, 3) == kd


def test_bsr_closed_forms(O):
    # banded half-bandwidth 64 at 8192: nnz = 8192*129 - 2*(64*65/2)
    M = 8192
    rows, cols = [], []
    for r in range(M):
        lo, hi = max(0, r - 64), min(M, r + 65)
        rows.append(np.full(hi - lo, r, np.int32))
        cols.append(np.arange(lo, hi, dtype=np.int32))
    r, c = np.concatenate(rows), np.concatenate(cols)
    rp, ci, va = O.coo_to_csr(M, r, c, np.ones(r.size, np.float32))
    assert ci.size == 8192 * 129 - 64 * 65 == 1052608
    brp, bci, _ = O.bsr_build(M, M, rp, ci, va)
    fill, _, _ = O.bsr_stats(M, M, int(brp[-1]), ci.size)
    # block-row br touches block-cols max(0, br-4) .. min(511, br+4): 5, 6, 7, 8
    # at each edge, 9 in the interior
    assert int(brp[-1]) == 2 * (5 + 6 + 7 + 8) + 504 * 9 == 4588
    assert round(fill, 4) == 1.1158


def test_bsr_spmm_f32_exact_small_and_bounded(O):
    rng = np.random.default_rng(21)
    M, K, N = 45, 70, 24
    n = 600
    r = rng.integers(0, M, n)
    c = rng.integers(0, K, n)
    v = rng.uniform(-1, 1, n).astype(np.float32)
    rp, ci, va = O.coo_to_csr(M, r, c, v)
    brp, bci, bv = O.bsr_build(M, K, rp, ci, va)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    B16 = O.f32_to_f16(B)
    C = O.bsr_spmm_f32(M, K, brp, bci, bv, B16, threads=3)
    A16 = _dense_from_bsr(M, K, brp, bci, bv).astype(np.float64)
    Bh = B16.view(np.float16).astype(np.float64)
    exact = A16 @ Bh
    absb = np.abs(A16) @ np.abs(Bh)
    # fp32 accumulation of exact fp16 products: error <= K * u * |A||B|
    assert np.all(np.abs(C - exact) <= 70 * 2.0**-24 * absb + 1e-30)
    # identity blocks -> C == fp16(B) rows
    Mi = 32
    rp_i = np.arange(Mi + 1, dtype=np.int32)
    ci_i = np.arange(Mi, dtype=np.int32)
    brp, bci, bv = O.bsr_build(Mi, Mi, rp_i, ci_i, np.ones(Mi, np.float32))
    Bi = rng.uniform(-1, 1, (Mi, 16)).astype(np.float32)
    Ci = O.bsr_spmm_f32(Mi, Mi, brp, bci, bv, O.f32_to_f16(Bi))
    assert np.array_equal(Ci, Bi.astype(np.float16).astype(np.float32))


def test_hybrid_rule_table(O):
    # spmm_hybrid.cu:35-54: MFMA iff N % 16 == 0 and N > 0 and fill <= threshold
    cases = [((1.0, 128, 2.0), (1, 0)), ((2.0, 128, 2.0), (1, 0)),
             ((2.0000001, 128, 2.0), (0, 2)), ((92.4, 128, 2.0), (0, 2)),
             ((1.0, 100, 2.0), (0, 1)), ((1.0, 0, 2.0), (0, 1)), ((1.0, -16, 2.0), (0, 1)),
             ((1.1158, 128, 1.0), (0, 2)), ((0.0, 16, 2.0), (1, 0))]
    for args, want in cases:
        assert O.hybrid_rule(*args) == want, args


def _bounds_by_definition(rp, parts):
    M, total = rp.size - 1, int(rp[-1])
    out = [0]
    for g in range(1, parts):
        target = total * g // parts
        r = next((i for i in range(M) if rp[i] >= target), M)
        out.append(r)
    out.append(M)
    for g in range(1, parts + 1):
        out[g] = max(out[g], out[g - 1])
    return np.array(out, np.int32)


def test_nnz_balanced_bounds(O):
    rng = np.random.default_rng(4)
    for M in (1, 7, 300):
        deg = rng.integers(0, 40, M)
        deg[rng.integers(0, M)] = 500  # one long row
        rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
        for parts in (1, 2, 5, 64):
            b = O.nnz_balanced_bounds(rp, parts)
            assert np.array_equal(b, _bounds_by_definition(rp, parts))
            assert b[0] == 0 and b[-1] == M and np.all(np.diff(b) >= 0)
            per = rp[b[1:]] - rp[b[:-1]]
            assert per.max() <= -(-int(rp[-1]) // parts) + deg.max()


def test_metrics_hand_computed(O):
    ours = np.array([1.0, 2.0, 3.5, 0.0001], np.float32)
    ref = np.array([1.0, 2.5, 3.0, 0.0], np.float32)
    ma, mr, rl = O.compare(ours, ref)
    assert ma == np.float32(0.5)
    assert mr == pytest.approx(0.5 / 2.5, rel=1e-6)  # cell 3 is below the 1e-3*peak floor
    assert rl == pytest.approx(np.sqrt(0.5**2 * 2 + 1e-8) / np.sqrt(1 + 6.25 + 9), rel=1e-6)
    assert O.rel_l2(ours, ref) == pytest.approx(rl, rel=1e-6)
    assert O.median([3.0, 1.0, 2.0, 10.0]) == 3.0  # v[n/2] after sort
    assert O.median([5.0]) == 5.0
