"""Merge-path launch over B-row halves (the CSR form spmm_hybrid_run picks for
c5: B of 8 MiB, over one XCD's 4 MiB L2 at full width, half of it within).
Parity with the fp64 oracle on c5 and on small matrices built to reach every
path of the halves -- rows cut across many parts in both halves, empty rows,
rows whose entries all lie in one half, unsorted columns with repeats, odd K,
N = 4 .. 256 -- bitwise repeatability, and the plan's refusals."""
import numpy as np
import pytest

from gpu_util import check_csr, make_config

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _plan_run(S, torch, A, B):
    """Two launches of one plan on NaN-filled C: both bit-identical."""
    N = B.shape[1]
    with S.KHalfPlan(A, N) as p:
        dB = torch.from_numpy(B).cuda()
        C = torch.full((A.num_rows, N), float("nan"), device="cuda")
        p.launch(dB, C)
        torch.cuda.synchronize()
        C1 = C.cpu().numpy()
        C.fill_(float("nan"))
        p.launch(dB, C)
        torch.cuda.synchronize()
        C2 = C.cpu().numpy()
    assert np.array_equal(C1.view(np.int32), C2.view(np.int32)), "launches differ"
    return C1


def test_khalf_c5(S, O, torch):
    A, B = make_config(S, "c5")
    N = B.shape[1]
    assert S.csr_auto_form(A, N)[0] == "khalf"
    say(f"khalf config=c5 M={A.num_rows} K={A.num_cols} N={N} nnz={A.nnz}")
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    rel = check_csr(_plan_run(S, torch, A, B), C64, absC)
    say(f"  rel_l2={rel:.3e}")


def _mixed(S, M, K, seed):
    """Rows of every kind, columns unsorted with repeats: empty rows, rows in
    the lower or upper half only, short mixed rows and two long rows (3000 and
    6000 entries) that cross many parts of both halves."""
    rng = np.random.default_rng(seed)
    K0 = K // 2
    lens, cols = [], []
    for r in range(M):
        kind = r % 6
        if kind == 0:
            c = np.empty(0, np.int64)
        elif kind == 1:
            c = rng.integers(0, K0, size=rng.integers(1, 40))
        elif kind == 2:
            c = rng.integers(K0, K, size=rng.integers(1, 40))
        else:
            c = rng.integers(0, K, size=rng.integers(1, 80))
        if r == M // 3:
            c = rng.integers(0, K, size=3000)
        if r == M // 2:
            c = rng.integers(0, K, size=6000)
        if c.size > 3:
            c[1] = c[0]  # a repeated column
        lens.append(c.size)
        cols.append(c)
    row_ptr = np.zeros(M + 1, np.int32)
    row_ptr[1:] = np.cumsum(lens)
    col = np.concatenate(cols).astype(np.int32)
    val = rng.uniform(-1, 1, size=col.size).astype(np.float32)
    return S.HostCSR(M, K, row_ptr, col, val)


CASES = {
    # name: (M, K, N, seed); every K x N x 4 is over 4 MiB with half within
    "power_law_odd_K": ("power_law", 600, 12345, 128, 41),
    "mixed_N128": ("mixed", 1200, 10000, 128, 42),
    "mixed_N256": ("mixed", 900, 6001, 256, 43),
    "mixed_N64": ("mixed", 700, 20000, 64, 44),
    "mixed_N4": ("mixed", 2000, 300001, 4, 45),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_khalf_cases(S, O, torch, case):
    kind, M, K, N, seed = CASES[case]
    if kind == "power_law":
        A = S.generate_power_law_csr(M, K, 80.0, 1.5, 4000, seed)
    else:
        A = _mixed(S, M, K, seed)
    B = np.random.default_rng(seed + 1).uniform(-1, 1, size=(K, N)).astype(np.float32)
    say(f"khalf case={case} M={M} K={K} N={N} nnz={A.nnz}")
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    check_csr(_plan_run(S, torch, A, B), C64, absC)


def test_khalf_refusals(S, torch):
    A, B = make_config(S, "c5")
    # N % 4 != 0, and a B that fits one L2 (c5 at N = 64: exactly 4 MiB)
    for N in (6, 64):
        with pytest.raises(S.SpmmError) as e:
            S.KHalfPlan(A, N)
        assert e.value.code == S.SPMM_UNSUPPORTED
    # a half with fewer than 512 entries
    few = S.HostCSR(4, 16384, np.array([0, 600, 600, 700, 700], np.int32),
                    np.r_[np.arange(600), 8192 + np.arange(100)].astype(np.int32),
                    np.ones(700, np.float32))
    with pytest.raises(S.SpmmError) as e:
        S.KHalfPlan(few, 128)
    assert e.value.code == S.SPMM_UNSUPPORTED
    # a column outside [0, K)
    bad = S.HostCSR(1, 16384, np.array([0, 2], np.int32), np.array([3, 16384], np.int32),
                    np.ones(2, np.float32))
    with pytest.raises(S.SpmmError) as e:
        S.KHalfPlan(bad, 128)
    assert e.value.code == S.SPMM_INVALID
    N = B.shape[1]
    p = S.KHalfPlan(A, N)
    dB = torch.from_numpy(B).cuda()
    # C 4 bytes off a 16-byte boundary
    buf = torch.empty(A.num_rows * N + 1, device="cuda")
    with pytest.raises(S.SpmmError) as e:
        p.launch(dB, buf[1:].view(A.num_rows, N))
    assert e.value.code == S.SPMM_UNSUPPORTED
    with pytest.raises(S.SpmmError) as e:  # B of the wrong width
        p.launch(dB[:, :64].contiguous())
    assert e.value.code == S.SPMM_INVALID
    p.close()
    with pytest.raises(S.SpmmError):
        p.launch(dB)
