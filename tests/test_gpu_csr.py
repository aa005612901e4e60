"""GPU parity of the seven CSR entry points (roles of src/kernels/spmm_*.cu)
against the fp64 oracle, through the C ABI on cuda:0.

Bar (north star): fp32 output within 1e-5 relative of the fp64-accumulated host
loop -- elementwise relative to (|A||B|)_ij and normwise (gpu_util.check_csr).
Every output buffer is pre-filled with NaN so an unwritten element fails.
"""
import ctypes

import numpy as np
import pytest

from gpu_util import check_csr, make_config

pytestmark = pytest.mark.gpu

KERNELS = ("baseline", "memopt", "memopt_v2", "tiled", "tiled_v2", "tiled_v3", "tiled_v4")


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _coo_csr(S, M, K, r, c, v):
    return S.csr_from_coo_host(M, K, np.asarray(r), np.asarray(c), np.asarray(v, np.float32))


def _edge_cases(S):
    rng = np.random.default_rng(1234)
    cases = {}
    cases["empty_nnz"] = (S.csr_from_coo_host(37, 50, [], [], []), rng.uniform(-1, 1, (50, 128)))
    cases["one_by_one"] = (_coo_csr(S, 1, 1, [0], [0], [0.75]), np.array([[2.0]]))
    cases["k_is_1"] = (_coo_csr(S, 40, 1, np.arange(0, 40, 3), np.zeros(14, int),
                                rng.uniform(-1, 1, 14)), rng.uniform(-1, 1, (1, 64)))
    ident = 300
    cases["identity"] = (_coo_csr(S, ident, ident, np.arange(ident), np.arange(ident),
                                  np.ones(ident)), rng.uniform(-1, 1, (ident, 128)))
    # empty rows, one long row (3000 entries), duplicates
    M, K = 500, 4000
    r = list(rng.integers(0, M, 6000))
    c = list(rng.integers(0, K, 6000))
    r += [7] * 3000
    c += list(rng.permutation(K)[:3000])
    r += [11, 11, 11]
    c += [5, 5, 5]
    keep = [i for i in range(len(r)) if r[i] % 5 != 3]  # every fifth row empty
    v = rng.uniform(-1, 1, len(keep))
    cases["ragged"] = (_coo_csr(S, M, K, np.array(r)[keep], np.array(c)[keep], v),
                       rng.uniform(-1, 1, (K, 128)))
    # the same rows at N = 520: each wave's range spans several LDS windows
    # (the 3000-entry row) and every window is walked in three column passes
    cases["ragged_wide"] = (cases["ragged"][0], rng.uniform(-1, 1, (K, 520)))
    for N in (1, 3, 17, 20, 32, 64, 96, 130, 256, 257, 512, 4100):
        A = S.generate_uniform_random_csr(200, 300, 0.05, N)
        cases[f"n{N}"] = (A, rng.uniform(-1, 1, (300, N)))
    # power-law rows at a small size: 2 .. 2000 entries per row
    A = S.generate_power_law_csr(1000, 3000, 60.0, 1.5, 2000, 77)
    cases["power_law_small"] = (A, rng.uniform(-1, 1, (3000, 128)))
    return cases


@pytest.fixture(scope="module")
def edge_cases(S, O):
    out = {}
    for name, (A, B) in _edge_cases(S).items():
        B = np.ascontiguousarray(B, np.float32)
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
        out[name] = (A, B, C64, absC)
    return out


def _run(S, torch, kernel, A, B):
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    dC = torch.full((A.num_rows, B.shape[1]), float("nan"), dtype=torch.float32, device="cuda")
    S.spmm_csr(kernel, dA, dB, dC)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


@pytest.mark.parametrize("kernel", KERNELS)
def test_edge_cases(S, torch, edge_cases, kernel):
    for name, (A, B, C64, absC) in edge_cases.items():
        if kernel == "tiled_v2" and B.shape[1] % 128 != 0:
            continue  # contract: N % 128 == 0 (tested separately)
        say(f"csr {kernel} case={name} M={A.num_rows} K={A.num_cols} N={B.shape[1]} nnz={A.nnz}")
        C = _run(S, torch, kernel, A, B)
        check_csr(C, C64, absC)


@pytest.fixture(scope="module")
def config_refs(S, O):
    cache = {}

    def get(name):
        if name not in cache:
            A, B = make_config(S, name)
            C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
            cache[name] = (A, B, C64, absC)
        return cache[name]
    return get


@pytest.mark.parametrize("cfg", ["c1", "c2", "c5"])
@pytest.mark.parametrize("kernel", KERNELS)
def test_configs(S, torch, config_refs, kernel, cfg):
    A, B, C64, absC = config_refs(cfg)
    say(f"csr {kernel} config={cfg} M={A.num_rows} N={B.shape[1]} nnz={A.nnz}")
    C = _run(S, torch, kernel, A, B)
    rel = check_csr(C, C64, absC)
    say(f"  rel_l2={rel:.3e}")


@pytest.mark.parametrize("kernel", ["baseline", "memopt", "memopt_v2"])
def test_sequential_roles_are_the_reference_chain_bit_for_bit(S, O, torch, edge_cases,
                                                               config_refs, kernel):
    # spmm_baseline, spmm_memopt and spmm_memopt_v2 (spmm_baseline.cu:11-25,
    # spmm_memopt.cu:17-37, spmm_memopt_v2.cu) each compute an output as
    # sum += value * b from 0.f in CSR order, one fused multiply-add per entry
    # under nvcc's default contraction; they differ only in how threads map to
    # outputs. The lane-per-output and wave-per-row kernels compute the same
    # chain, so their results equal the CPU restatement bit for bit.
    cases = [(name, A, B) for name, (A, B, _, _) in edge_cases.items()]
    A, B, _, _ = config_refs("c1")
    cases.append(("c1", A, B))
    for name, A, B in cases:
        say(f"csr {kernel} bitwise case={name} M={A.num_rows} N={B.shape[1]} nnz={A.nnz}")
        C = _run(S, torch, kernel, A, B)
        ref = O.csr_spmm_f32_fma(A.row_ptr, A.col_idx, A.values, B)
        assert np.array_equal(C.view(np.uint32), ref.view(np.uint32)), name


@pytest.mark.parametrize("cfg", ["c1", "c2"])
def test_row_groups_one_entry_lane_is_the_reference_chain(S, O, torch, config_refs, cfg):
    # The tiled roles' fast forms associate a row's sum differently from the
    # reference's fused chain. The row groups with one entry lane per row do
    # not: each lane sums its columns over the row's entries in CSR order
    # with fused multiply-adds, so the option reproduces the reference kernels
    # bit for bit (for rows that stay in their group, as all of c1's and c2's do).
    A, B, _, _ = config_refs(cfg)
    opts = S.EngineOptsT()
    opts.row_groups = 1
    opts.entry_lanes = 1
    opts.unroll = 4  # four entries in flight per lane (same order, faster)
    say(f"csr row groups, one entry lane, bitwise config={cfg}")
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    dC = torch.full((A.num_rows, B.shape[1]), float("nan"), dtype=torch.float32, device="cuda")
    S.launch_repeat_opts(dA, dB, dC, opts, 1)
    torch.cuda.synchronize()
    ref = O.csr_spmm_f32_fma(A.row_ptr, A.col_idx, A.values, B)
    assert np.array_equal(dC.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("cfg", ["c3", "c4"])
def test_engine_on_fp16_configs(S, torch, config_refs, cfg):
    # the CSR back end must also be right on the structured configs: the
    # dispatcher compares both back ends there
    A, B, C64, absC = config_refs(cfg)
    say(f"csr tiled_v3 config={cfg}")
    check_csr(_run(S, torch, "tiled_v3", A, B), C64, absC)


def test_engine_deterministic(S, torch, config_refs):
    A, B, _, _ = config_refs("c5")
    say("csr tiled_v3 determinism c5")
    c1 = _run(S, torch, "tiled_v3", A, B)
    c2 = _run(S, torch, "tiled_v3", A, B)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))


@pytest.mark.parametrize("vec", [1, 2, 4])
@pytest.mark.parametrize("groups", [1, 2, 4, 8])
@pytest.mark.parametrize("waves,unroll,gl", [(2, 8, 0), (4, 4, 0), (8, 8, 0), (8, 4, 1)])
def test_engine_variants(S, torch, edge_cases, config_refs, vec, groups, waves, unroll, gl):
    # gl = 1: B through 64-bit address loads (the form used when B does not
    # fit a buffer resource) instead of structured-buffer loads
    opts = S.EngineOptsT(vec, waves, unroll, 0, groups, 0, gl)
    for name in ("ragged", "ragged_wide", "power_law_small", "n3", "n17", "n20", "n32", "n96",
                 "n257", "n512", "n4100", "empty_nnz"):
        A, B, C64, absC = edge_cases[name]
        say(f"csr engine vec={vec} groups={groups} waves={waves} unroll={unroll} gl={gl} case={name}")
        dA = S.DeviceCSR(A)
        dB = torch.from_numpy(B).cuda()
        dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
        S.spmm_tiled_v3_opts(dA, dB, opts, dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)
    for rpb in (1, 7, 1024):
        A, B, C64, absC = edge_cases["ragged"]
        say(f"csr engine vec={vec} groups={groups} waves={waves} unroll={unroll} gl={gl} rows_per_block={rpb}")
        dA = S.DeviceCSR(A)
        dB = torch.from_numpy(B).cuda()
        dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
        S.spmm_tiled_v3_opts(dA, dB, S.EngineOptsT(vec, waves, unroll, rpb, groups, 0, gl), dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)


@pytest.mark.parametrize("slices", [2, 4, 8])
@pytest.mark.parametrize("vec", [0, 1])
def test_engine_column_slices(S, torch, edge_cases, config_refs, slices, vec):
    opts = S.EngineOptsT(vec, 8, 4, 0, 0, slices)
    for name in ("ragged", "ragged_wide", "power_law_small", "n1", "n3", "n17", "n96", "n130",
                 "n257", "n512", "empty_nnz", "identity"):
        A, B, C64, absC = edge_cases[name]
        say(f"csr engine slices={slices} vec={vec} case={name}")
        dA = S.DeviceCSR(A)
        dB = torch.from_numpy(B).cuda()
        dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
        S.spmm_tiled_v3_opts(dA, dB, opts, dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)
    A, B, C64, absC = config_refs("c5")
    say(f"csr engine slices={slices} vec={vec} config=c5")
    dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
    S.spmm_tiled_v3_opts(S.DeviceCSR(A), torch.from_numpy(B).cuda(), opts, dC)
    torch.cuda.synchronize()
    check_csr(dC.cpu().numpy(), C64, absC)


@pytest.mark.parametrize("parts", [1, 3, 64, 5000])
def test_partitioned_engine(S, torch, edge_cases, config_refs, parts):
    cases = [edge_cases["ragged"], edge_cases["power_law_small"], config_refs("c5")]
    for A, B, C64, absC in cases:
        say(f"csr partitioned parts={parts} M={A.num_rows} nnz={A.nnz}")
        bounds = torch.from_numpy(S.nnz_balanced_bounds(A, parts)).cuda()
        dA = S.DeviceCSR(A)
        dB = torch.from_numpy(B).cuda()
        dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
        S.spmm_tiled_v3_partitioned(dA, bounds, dB, dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)


def _split_run(S, torch, A, B, parts):
    rows = torch.from_numpy(S.nnz_split_rows(A, parts)).cuda()
    dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
    S.spmm_tiled_v3_split(S.DeviceCSR(A), rows, torch.from_numpy(B).cuda(), dC)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


@pytest.mark.parametrize("parts", [1, 2, 7, 64, 513, 5000])
def test_split_engine(S, torch, edge_cases, config_refs, parts):
    # merge-path partition: equal nonzero ranges per workgroup, rows cut
    # between workgroups and completed by the carry fix-up
    names = ("ragged", "ragged_wide", "power_law_small", "identity", "k_is_1", "n1", "n3", "n17",
             "n96", "n130", "n257", "n512", "one_by_one")
    for name in names:
        A, B, C64, absC = edge_cases[name]
        p = max(1, min(parts, A.nnz))
        say(f"csr split parts={p} case={name} M={A.num_rows} nnz={A.nnz} N={B.shape[1]}")
        check_csr(_split_run(S, torch, A, B, p), C64, absC)
    A, B, C64, absC = config_refs("c5")
    say(f"csr split parts={parts} config=c5")
    check_csr(_split_run(S, torch, A, B, parts), C64, absC)


def test_split_engine_long_rows_and_empty_rows(S, O, torch):
    # one row of 20000 entries spanning dozens of parts, empty rows on part
    # boundaries and at both ends, a part of a single nonzero
    rng = np.random.default_rng(21)
    M, K, N = 300, 30000, 64
    r = [5] * 20000 + list(rng.integers(10, 290, 3000)) + [299]
    c = list(rng.permutation(K)[:20000]) + list(rng.integers(0, K, 3000)) + [7]
    keep = [i for i in range(len(r)) if r[i] % 4 != 1]
    A = S.csr_from_coo_host(M, K, np.array(r)[keep], np.array(c)[keep],
                            rng.uniform(-1, 1, len(keep)).astype(np.float32))
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
    for parts in (3, 40, 333, A.nnz):
        say(f"csr split long-row parts={parts} nnz={A.nnz}")
        C1 = _split_run(S, torch, A, B, parts)
        check_csr(C1, C64, absC)
        C2 = _split_run(S, torch, A, B, parts)
        assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))  # deterministic


def test_split_engine_errors(S, torch):
    s = S.CsrT(4, 4, 1, 0, 0, 0)
    assert S.lib().spmm_c_tiled_v3_split(ctypes.byref(s), None, 1, 0, 0, 4, None, None) == \
        S.SPMM_INVALID
    # more parts than nonzeros (an empty part) is refused before any launch
    A = S.csr_from_coo_host(4, 4, [0, 0, 1], [0, 1, 2], [1.0, 2.0, 3.0])
    dA = S.DeviceCSR(A)
    B = torch.ones((4, 8), device="cuda")
    rows = torch.zeros(5, dtype=torch.int32, device="cuda")  # 4 parts > 3 nonzeros
    with pytest.raises(S.SpmmError) as e:
        S.spmm_tiled_v3_split(dA, rows, B)
    assert e.value.code == S.SPMM_INVALID
    assert "parts <= max(nnz, 1)" in str(e.value)
    # parts == nnz is the largest accepted split
    C = S.spmm_tiled_v3_split(dA, torch.from_numpy(S.nnz_split_rows(A, 3)).cuda(), B)
    torch.cuda.synchronize()
    assert np.allclose(C.cpu().numpy(), A.to_dense() @ np.ones((4, 8), np.float32))


def test_tiled_v2_contract(S, torch, edge_cases):
    A, B, _, _ = edge_cases["n96"]
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    with pytest.raises(S.SpmmError) as e:
        S.spmm_csr("tiled_v2", dA, dB)
    assert e.value.code == S.SPMM_UNSUPPORTED
    assert "N % 128" in str(e.value)


def _run_opts(S, torch, A, B, opts):
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    dC = torch.full((A.num_rows, B.shape[1]), float("nan"), device="cuda")
    S.spmm_tiled_v3_opts(dA, dB, opts, dC)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


@pytest.mark.parametrize("form", [1, 2, 3])
@pytest.mark.parametrize("vec", [0, 1, 2])
@pytest.mark.parametrize("entry_lanes,unroll", [(0, 0), (1, 2), (4, 4), (64, 2)])
def test_row_groups(S, torch, edge_cases, form, vec, entry_lanes, unroll):
    # sub-wave row groups on every edge case: empty rows, duplicates, rows far
    # longer than a group's share (the wave-wide pass), N from 1 to 520; form
    # 2 = per-lane index loads, 3 = cooperative index loads, 1 = chosen
    opts = S.EngineOptsT(vec, 0, unroll, 0, 0, 0, 0, form, entry_lanes)
    for name, (A, B, C64, absC) in edge_cases.items():
        say(f"csr row groups form={form} vec={vec} entry_lanes={entry_lanes} unroll={unroll} "
            f"case={name}")
        if B.shape[1] * 4 > 16383:
            with pytest.raises(S.SpmmError):  # a B row no longer fits one buffer record
                _run_opts(S, torch, A, B, opts)
            continue
        check_csr(_run_opts(S, torch, A, B, opts), C64, absC)


@pytest.mark.parametrize("form", [1, 2, 3])
def test_row_groups_max_row_hint(S, torch, edge_cases, form):
    # with the true longest row as a hint the kernel drops its long-row pass
    # whenever no row needs it (and keeps it otherwise); results are the same
    for name, (A, B, C64, absC) in edge_cases.items():
        if B.shape[1] * 4 > 16383:
            continue
        hint = int(np.diff(A.row_ptr).max()) if A.num_rows else 0
        say(f"csr row groups max_row_hint={hint} form={form} case={name}")
        opts = S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, form, 0, max(hint, 1))
        check_csr(_run_opts(S, torch, A, B, opts), C64, absC)


@pytest.mark.parametrize("form", [1, 2, 3])
def test_row_groups_undersized_hint(S, O, torch, form):
    # A hint below the true longest row drops the workgroup-wide long-row
    # pass; each group then sums its long row itself: slower, same result.
    # Rows of 2 entries with 3% long rows (up to K entries, a 4096-entry one).
    rng = np.random.default_rng(91)
    M, K, N = 3000, 4096, 32
    lens = np.where(rng.random(M) < 0.03, rng.integers(200, K + 1, M), 2)
    lens[17] = K
    rows = np.repeat(np.arange(M), lens)
    cols = np.concatenate([rng.choice(K, n, replace=False) for n in lens])
    A = S.csr_from_coo_host(M, K, rows, cols, rng.uniform(-1, 1, rows.size).astype(np.float32))
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
    for hint in (1, 2, 64, K):
        say(f"csr row groups undersized hint={hint} (true {K}) form={form}")
        opts = S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, form, 0, hint)
        check_csr(_run_opts(S, torch, A, B, opts), C64, absC)


@pytest.mark.parametrize("hint_kind", ["true", "average", "one"])
def test_engine_whole_round_grid(S, O, torch, edge_cases, hint_kind):
    # the row-block engine with a longest-row hint: rows within 2 x average +
    # 32 take the grid of whole rounds of 4-wave workgroups (1 .. kRpCap rows
    # per workgroup, 1 / 2 / 4 column slices); the hint only chooses the grid,
    # so a hint below the true longest row (power-law rows, ragged edge
    # cases) must give the same results as the true one
    for name, (A, B, C64, absC) in edge_cases.items():
        if A.num_rows == 0 or A.nnz == 0:
            continue
        lens = np.diff(A.row_ptr)
        hint = {"true": int(lens.max()), "average": max(1, A.nnz // A.num_rows), "one": 1}[hint_kind]
        say(f"csr engine whole-round hint={hint} ({hint_kind}) case={name}")
        opts = S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, 0, 0, hint)
        check_csr(_run_opts(S, torch, A, B, opts), C64, absC)
    rng = np.random.default_rng(17)
    shapes = [(1, 300, 16, 128), (1000, 2048, 8, 64), (4096, 4096, 41, 128), (12288, 12288, 5, 128),
              (9000, 20000, 3, 256), (70000, 4096, 2, 8)]
    for M, K, avg, N in shapes:
        A = S.generate_uniform_random_csr(M, K, min(1.0, avg / K), 100 + M)
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
        lens = np.diff(A.row_ptr)
        hint = {"true": int(lens.max()), "average": max(1, A.nnz // M), "one": 1}[hint_kind]
        say(f"csr engine whole-round hint={hint} ({hint_kind}) M={M} K={K} N={N} nnz={A.nnz}")
        opts = S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, 0, 0, hint)
        check_csr(_run_opts(S, torch, A, B, opts), C64, absC)
    A = S.generate_power_law_csr(8192, 8192, 64.0, 1.5, 2048, 9)
    B = rng.uniform(-1, 1, (8192, 128)).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
    hint = {"true": int(np.diff(A.row_ptr).max()), "average": A.nnz // 8192, "one": 1}[hint_kind]
    say(f"csr engine whole-round hint={hint} ({hint_kind}) power-law nnz={A.nnz}")
    check_csr(_run_opts(S, torch, A, B, S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, 0, 0, hint)), C64, absC)


@pytest.mark.parametrize("N", [8, 12, 16, 24, 32, 40])
def test_default_narrow_b(S, O, torch, N):
    # plain spmm_tiled_v3 / _v4 at narrow B: row groups by default up to four
    # 16-byte column lanes, and up to eight on up to 4 M nonzeros (the
    # engine above that and for N = 40); tall uniform and power-law matrices
    rng = np.random.default_rng(60 + N)
    mats = [S.generate_uniform_random_csr(70000, 4096, 6.0 / 4096, 61),
            S.generate_power_law_csr(20000, 20000, 30.0, 1.5, 4096, 62)]
    for A in mats:
        B = rng.uniform(-1, 1, (A.num_cols, N)).astype(np.float32)
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
        for kernel in ("tiled_v3", "tiled_v4"):
            say(f"csr default narrow {kernel} M={A.num_rows} K={A.num_cols} N={N} nnz={A.nnz}")
            dA = S.DeviceCSR(A)
            dC = torch.full((A.num_rows, N), float("nan"), device="cuda")
            S.spmm_csr(kernel, dA, torch.from_numpy(B).cuda(), dC)
            torch.cuda.synchronize()
            check_csr(dC.cpu().numpy(), C64, absC)


@pytest.mark.parametrize("slices", [2, 4, 8])
def test_row_groups_column_slices(S, torch, edge_cases, slices):
    # XCD-tied column slices: each workgroup computes 1/slices of the columns
    # (slices wider than N leave the later workgroups without columns)
    for form in (2, 3):
        opts = S.EngineOptsT(0, 0, 0, 0, 0, slices, 0, form, 0)
        for name, (A, B, C64, absC) in edge_cases.items():
            if B.shape[1] * 4 > 16383:
                continue
            say(f"csr row groups slices={slices} form={form} case={name}")
            check_csr(_run_opts(S, torch, A, B, opts), C64, absC)


@pytest.mark.parametrize("form", [2, 3])
@pytest.mark.parametrize("entry_lanes,unroll", [(8, 2), (2, 4), (16, 4)])
def test_row_groups_long_row_boundary(S, O, torch, form, entry_lanes, unroll):
    # N = 16 (four column lanes of 4 floats): a row longer than
    # 8 * entry_lanes * unroll entries (and 4x the average row, which the
    # 300 one-entry rows keep below that) moves to the wave-wide pass; rows of
    # that length -1 / +0 / +1 / x2, several long rows in one wave, empty rows,
    # and a row count that is not a multiple of the rows per workgroup
    rng = np.random.default_rng(entry_lanes * 10 + unroll)
    cut = 8 * entry_lanes * unroll
    lens = [cut - 1, cut, cut + 1, 2 * cut, cut + 1, 0, 3, cut + 5, 0, 2 * cut + 7, 1] * 3 + [cut + 2]
    lens += [1] * 300
    assert 4.0 * sum(lens) / len(lens) < cut
    K = 4 * cut + 50
    rows, cols = [], []
    for r, n in enumerate(lens):
        rows += [r] * n
        cols += list(rng.choice(K, n, replace=False))
    A = _coo_csr(S, len(lens), K, rows, cols, rng.uniform(-1, 1, len(rows)))
    B = rng.uniform(-1, 1, (K, 16)).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
    say(f"csr row groups long-row boundary form={form} cut={cut} rows={len(lens)}")
    C = _run_opts(S, torch, A, B, S.EngineOptsT(4, 0, unroll, 0, 0, 0, 0, form, entry_lanes))
    check_csr(C, C64, absC)


@pytest.mark.parametrize("N", [1, 4, 16, 64])
def test_row_groups_c2_narrow(S, O, torch, N):
    # the c2 matrix at narrow B, where row groups are the hybrid's CSR choice;
    # results are bitwise identical run to run
    A, _ = make_config(S, "c2")
    B = np.random.default_rng(N).uniform(-1, 1, (A.num_cols, N)).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    opts = S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, 1, 0)
    say(f"csr row groups c2 N={N}")
    C1 = _run_opts(S, torch, A, B, opts)
    check_csr(C1, C64, absC)
    C2 = _run_opts(S, torch, A, B, opts)
    assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))


@pytest.mark.parametrize("N", [64, 128, 256])
def test_row_groups_tall(S, O, torch, N):
    # 32768 rows: the column lanes drop to 16 (several column passes), the
    # entry lanes follow the wave target and the cooperative loads are chosen
    A = S.generate_uniform_random_csr(32768, 32768, 16.0 / 32768, 91)
    B = np.random.default_rng(N + 1).uniform(-1, 1, (32768, N)).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    for form in (1, 2, 3):
        say(f"csr row groups tall M=32768 N={N} form={form}")
        check_csr(_run_opts(S, torch, A, B, S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, form, 0)),
                  C64, absC)


def test_row_groups_argument_errors(S, torch, edge_cases):
    A, B, _, _ = edge_cases["ragged"]
    for lanes in (3, -2, 128):  # entry lanes: a power of two up to 64
        with pytest.raises(S.SpmmError):
            _run_opts(S, torch, A, B, S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, 1, lanes))
    for form in (-1, 4):  # 0 engine, 1 chosen, 2 per-lane loads, 3 cooperative loads
        with pytest.raises(S.SpmmError):
            _run_opts(S, torch, A, B, S.EngineOptsT(0, 0, 0, 0, 0, 0, 0, form, 0))


def test_launch_argument_errors(S, torch):
    s = S.CsrT(4, 4, 2, 0, 0, 0)  # nnz > 0 but null arrays
    rc = S.lib().spmm_c_tiled_v3(ctypes.byref(s), 1, 1, 8, None)
    assert rc == S.SPMM_INVALID
    s = S.CsrT(-1, 4, 0, 0, 0, 0)
    assert S.lib().spmm_c_baseline(ctypes.byref(s), 0, 0, 8, None) == S.SPMM_INVALID
    s = S.CsrT(4, 4, 0, 0, 0, 0)  # N == 0: nothing to do
    assert S.lib().spmm_c_memopt(ctypes.byref(s), 0, 0, 0, None) == S.SPMM_OK


def test_size_independent_properties_c2(S, torch, config_refs):
    # linearity in B and scaling by powers of two hold exactly-or-nearly at full size
    A, B, _, _ = config_refs("c2")
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    say("csr tiled_v3 linearity c2")
    c1 = S.spmm_csr("tiled_v3", dA, dB)
    c2 = S.spmm_csr("tiled_v3", dA, dB * 4.0)
    assert torch.equal(c2, c1 * 4.0)  # power-of-two scaling is exact
    c3 = S.spmm_csr("tiled_v3", dA, dB + dB)
    assert torch.equal(c3, c1 * 2.0)
    neg = S.spmm_csr("tiled_v3", dA, -dB)
    assert torch.equal(neg, -c1)
