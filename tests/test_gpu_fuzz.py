"""Seeded random parity sweep on cuda:0: random shapes, densities, row-length
skew and engine options for the CSR engine (row partition, merge-path, merge-path
over B-row halves and the sub-wave row groups, the latter also with their own
load forms, slices and longest-row hints), and random shapes and kernel options for the MFMA BSR
kernel, each checked against the CPU oracle with the same bars as the other
GPU tests (fp32 CSR within 1e-5 of the fp64 loop; fp16 BSR within 1e-2 of
fp32 accumulation and within 1e-5 of the exact product of the fp16
operands)."""
import numpy as np
import pytest

from gpu_util import check_bsr, check_csr

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _skewed_csr(S, rng, M, K):
    """Rows of very different lengths (empty rows included), unique columns per row."""
    rows, cols = [], []
    for r in range(M):
        u = rng.random()
        if u < 0.2:
            n = 0
        elif u < 0.9:
            n = int(rng.integers(1, max(2, min(K, 40))))
        else:
            n = int(rng.integers(1, K + 1))  # up to a full row
        if n:
            rows.append(np.full(n, r))
            cols.append(rng.choice(K, n, replace=False))
    if not rows:
        return S.csr_from_coo_host(M, K, [], [], [])
    r = np.concatenate(rows)
    c = np.concatenate(cols)
    return S.csr_from_coo_host(M, K, r, c, rng.uniform(-1, 1, r.size).astype(np.float32))


def _random_csr(S, rng, M, K):
    kind = int(rng.integers(0, 3))
    if kind == 0:
        return S.generate_uniform_random_csr(M, K, float(rng.uniform(0.0, 0.15)),
                                             int(rng.integers(1, 10000)))
    if kind == 1:
        mean = float(rng.uniform(1.0, max(1.5, min(K, 60))))
        return S.generate_power_law_csr(M, K, mean, 1.5, K, int(rng.integers(1, 10000)))
    return _skewed_csr(S, rng, M, K)


def _shape(rng):
    M = int(rng.integers(1, 600))
    K = int(rng.integers(1, 800))
    N = int(rng.choice([1, 2, 3, 4, 8, 16, 20, 31, 32, 48, 64, 100, 128, 130, 192, 256, 300]))
    return M, K, N


@pytest.mark.parametrize("chunk", range(10))
def test_csr_engine_random(S, O, torch, chunk):
    rng = np.random.default_rng(1000 + chunk)
    hint_rng = np.random.default_rng(5000 + chunk)
    for case in range(30):
        M, K, N = _shape(rng)
        A = _random_csr(S, rng, M, K)
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        opts = S.EngineOptsT(int(rng.choice([0, 1, 2, 4])), int(rng.choice([0, 2, 4, 8])),
                             int(rng.choice([0, 2, 4, 8])),
                             int(rng.choice([0, 0, 1, 3, 16, 64])),
                             int(rng.choice([0, 1, 2, 4, 8])), int(rng.choice([0, 1, 2, 4, 8])),
                             int(rng.choice([0, 0, 1])), int(rng.choice([0, 0, 1, 2, 3])),
                             int(rng.choice([0, 1, 2, 8, 64])))
        # a longest-row hint from its own stream (the draws above stay as they
        # were): true, above it, or -- for the engine only, where it just
        # chooses the grid -- below it
        longest = int(np.diff(A.row_ptr).max()) if M and A.nnz else 0
        kinds = ["none", "true", "high"] + (["low"] if opts.row_groups == 0 else [])
        kind = kinds[int(hint_rng.integers(0, len(kinds)))]
        opts.max_row_hint = {"none": 0, "true": longest, "high": 2 * longest + 40,
                             "low": 1}[kind]
        say(f"fuzz csr chunk={chunk} case={case} M={M} K={K} N={N} nnz={A.nnz} "
            f"hint={kind}:{opts.max_row_hint} "
            f"opts=({opts.vec},{opts.waves},{opts.unroll},{opts.rows_per_block},{opts.groups},"
            f"{opts.slices},{opts.global_loads},{opts.row_groups},{opts.entry_lanes})")
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
        dA = S.DeviceCSR(A)
        dB = torch.from_numpy(B).cuda()
        dC = torch.full((M, N), float("nan"), device="cuda")
        S.spmm_tiled_v3_opts(dA, dB, opts, dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)
        if A.nnz > 0 and case % 3 == 0:
            parts = int(rng.integers(1, A.nnz + 1))
            say(f"fuzz csr split chunk={chunk} case={case} parts={parts}")
            rows = torch.from_numpy(S.nnz_split_rows(A, parts)).cuda()
            dC.fill_(float("nan"))
            S.spmm_tiled_v3_split(dA, rows, dB, dC)
            torch.cuda.synchronize()
            check_csr(dC.cpu().numpy(), C64, absC)


@pytest.mark.parametrize("chunk", range(10))
def test_mfma_random(S, O, torch, chunk):
    rng = np.random.default_rng(2000 + chunk)
    for case in range(25):
        M, K, N = _shape(rng)
        shape = int(rng.integers(0, 5))
        if shape == 3:    # banded: neighbouring block-rows share block-columns
            A = S.generate_banded_csr(M, K, int(rng.integers(0, 80)), int(rng.integers(1, 10000)))
        elif shape == 4:  # block-diagonal, block sizes not multiples of 16 included
            A = S.generate_block_diagonal_csr(M, K, int(rng.integers(1, 100)),
                                              int(rng.integers(1, 10000)), 1.0)
        else:
            A = _random_csr(S, rng, M, K)
        A.values = S.round_to_fp16(A.values)
        B = S.round_to_fp16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
        hb = S.bsr_from_csr_host(A)
        B16 = O.f32_to_f16(B)
        C32 = O.bsr_spmm_f32(M, K, hb.row_ptr, hb.col_idx, hb.values, B16, threads=8)
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B16.view(np.float16)
                                   .astype(np.float32), threads=8)
        kernel = int(rng.choice([0, 1, 4, 8]))  # automatic, wave, panel R = 4 / 8
        if kernel == 1:
            opts = S.BsrOptsT(1, int(rng.choice([0, 1, 2, 4])), 1, int(rng.choice([0, 1, 2, 4])),
                              int(rng.choice([0, 1, 2])), addressing=int(rng.choice([0, 1])))
        else:
            opts = S.BsrOptsT(kernel, int(rng.choice([0, 4, 8])), 0, int(rng.choice([0, 2, 4])),
                              int(rng.choice([0, 1, 2])))
        say(f"fuzz mfma chunk={chunk} case={case} M={M} K={K} N={N} blocks={hb.num_blocks} "
            f"opts=(row_group {opts.row_group}, tiles {opts.tiles}, depth {opts.depth}, "
            f"order {opts.xcd_order}, addressing {opts.addressing})")
        dC = torch.full((M, N), float("nan"), device="cuda")
        S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(), opts, dC)
        torch.cuda.synchronize()
        C = dC.cpu().numpy()
        check_bsr(C, C32, absC)
        check_csr(C, C64, absC, tol=1e-5)


def _long_row_csr(S, rng, M, K):
    """Mostly rows of 0-4 entries with ~3% rows of up to K entries."""
    rows, cols = [], []
    for r in range(M):
        n = int(rng.integers(0, 5)) if rng.random() < 0.97 else int(rng.integers(1, K + 1))
        if n:
            rows.append(np.full(n, r))
            cols.append(rng.choice(K, n, replace=False))
    if not rows:
        return S.csr_from_coo_host(M, K, [], [], [])
    r = np.concatenate(rows)
    c = np.concatenate(cols)
    return S.csr_from_coo_host(M, K, r, c, rng.uniform(-1, 1, r.size).astype(np.float32))


@pytest.mark.parametrize("chunk", range(5))
def test_row_groups_random(S, O, torch, chunk):
    # the sub-wave row groups under random shapes, skew, load forms, column
    # slices, entry lanes, unroll and longest-row hints (exact, above, and
    # below the true longest row: an under-sized hint drops the workgroup-wide
    # long-row pass, so each group sums its long row itself), plus the default
    # launch (row groups for N <= 32)
    rng = np.random.default_rng(3000 + chunk)
    for case in range(40):
        M = int(rng.integers(1, 1500))
        K = int(rng.integers(1, 1500))
        N = int(rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 24, 32, 40, 64, 96, 128, 160, 256]))
        A = _long_row_csr(S, rng, M, K) if rng.random() < 0.3 else _random_csr(S, rng, M, K)
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        mx = int(np.diff(A.row_ptr).max())
        opts = S.EngineOptsT(int(rng.choice([0, 1, 2, 4])), 0, int(rng.choice([0, 2, 4])), 0, 0,
                             int(rng.choice([0, 1, 2, 4, 8])), 0, int(rng.choice([1, 2, 3])),
                             int(rng.choice([0, 1, 2, 4, 8, 16, 64])),
                             int(rng.choice([0, mx, mx + 5, max(1, mx // 3), 1])))
        say(f"fuzz row groups chunk={chunk} case={case} M={M} K={K} N={N} nnz={A.nnz} max={mx} "
            f"opts=({opts.vec},{opts.unroll},{opts.slices},{opts.row_groups},{opts.entry_lanes},"
            f"{opts.max_row_hint})")
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
        dA = S.DeviceCSR(A)
        dB = torch.from_numpy(B).cuda()
        dC = torch.full((M, N), float("nan"), device="cuda")
        S.spmm_tiled_v3_opts(dA, dB, opts, dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)
        dC.fill_(float("nan"))
        S.spmm_csr("tiled_v3", dA, dB, dC)
        torch.cuda.synchronize()
        check_csr(dC.cpu().numpy(), C64, absC)


def _halves_csr(S, rng, M, K):
    """Rows of mixed lengths (empty, short, a few long ones) with columns drawn
    over all of K or, for some rows, from one half only; unsorted, repeats
    allowed (the B-row halves keep each row's entry order within a half)."""
    lens = np.where(rng.random(M) < 0.2, 0, rng.integers(1, 60, size=M))
    long_rows = rng.random(M) < 0.02
    lens[long_rows] = rng.integers(500, 4000, size=int(long_rows.sum()))
    K0 = K // 2
    cols = []
    for r in range(M):
        side = rng.random()
        lo, hi = (0, K0) if side < 0.15 else ((K0, K) if side < 0.3 else (0, K))
        cols.append(rng.integers(lo, hi, size=int(lens[r])))
    row_ptr = np.zeros(M + 1, np.int32)
    row_ptr[1:] = np.cumsum(lens)
    col = np.concatenate(cols).astype(np.int32) if cols else np.zeros(0, np.int32)
    return S.HostCSR(M, K, row_ptr, col, rng.uniform(-1, 1, col.size).astype(np.float32))


@pytest.mark.parametrize("chunk", range(4))
def test_khalf_random(S, O, torch, chunk):
    # merge-path over B-row halves on random shapes that qualify (N % 4 == 0,
    # K x N x 4 bytes over 4 MiB with half of the rows within it); a plan with
    # a half under 512 entries is refused
    rng = np.random.default_rng(7000 + chunk)
    for case in range(10):
        N = int(rng.choice([4, 8, 12, 16, 32, 64, 128, 192, 256]))
        kmin, kmax = (1 << 20) // N + 1, (1 << 21) // N
        K = int(rng.integers(kmin, kmax + 1))
        M = int(rng.integers(1, 900))
        A = _halves_csr(S, rng, M, K)
        n0 = int((A.col_idx < K // 2).sum())
        say(f"fuzz khalf chunk={chunk} case={case} M={M} K={K} N={N} nnz={A.nnz} half0={n0}")
        if min(n0, A.nnz - n0) < 512:
            with pytest.raises(S.SpmmError) as e:
                S.KHalfPlan(A, N)
            assert e.value.code == S.SPMM_UNSUPPORTED
            continue
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
        with S.KHalfPlan(A, N) as p:
            dC = torch.full((M, N), float("nan"), device="cuda")
            p.launch(torch.from_numpy(B).cuda(), dC)
            torch.cuda.synchronize()
            check_csr(dC.cpu().numpy(), C64, absC)
