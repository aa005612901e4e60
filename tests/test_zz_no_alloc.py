"""The allocation-free merge-path entry point (spmm_c_tiled_v3_split_noalloc)
against the entry point it mirrors (spmm_c_tiled_v3_split with a caller
workspace), through the C ABI: two calls in a row, the second on a smaller
input, each bitwise equal to the workspace launch (the carries are added in
part order, so both are deterministic) and within the fp32 bar of the fp64
oracle.  Sizes beyond the 2^19-float workspace are refused before any launch.
"""
import ctypes

import numpy as np
import pytest

from gpu_util import check_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _noalloc(S):
    return S.lib().spmm_c_tiled_v3_split_noalloc  # the C ABI entry point, called directly


def _case(S, O, torch, fn, A, N, parts, seed):
    B = np.random.default_rng(seed).uniform(-1, 1, (A.num_cols, N)).astype(np.float32)
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    rows = torch.from_numpy(S.nnz_split_rows(A, parts)).cuda()
    want = S.spmm_tiled_v3_split(dA, rows, dB)  # caller-provided carry workspace
    got = torch.full((A.num_rows, N), float("nan"), device="cuda")
    s = dA.struct()
    stream = torch.cuda.current_stream().cuda_stream
    rc = fn(ctypes.byref(s), rows.data_ptr(), parts, dB.data_ptr(), got.data_ptr(), N, stream)
    assert rc == S.SPMM_OK, S.lib().spmm_c_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want), "no-alloc launch differs from the workspace launch"
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=8)
    check_csr(got.cpu().numpy(), C64, absC)


def test_noalloc_matches_workspace_launch_twice(S, O, torch):
    fn = _noalloc(S)
    big = S.generate_power_law_csr(6000, 5000, 120.0, 1.5, 3000, 71)
    print(f"no-alloc call 1: M={big.num_rows} nnz={big.nnz} N=128 parts=512", flush=True)
    _case(S, O, torch, fn, big, 128, 512, 72)
    small = S.generate_power_law_csr(700, 900, 40.0, 1.5, 800, 73)
    print(f"no-alloc call 2: M={small.num_rows} nnz={small.nnz} N=48 parts=37", flush=True)
    _case(S, O, torch, fn, small, 48, 37, 74)


def test_noalloc_rejects_oversize(S, torch):
    fn = _noalloc(S)
    A = S.generate_uniform_random_csr(64, 64, 0.5, 5)
    dA = S.DeviceCSR(A)
    parts = 1024
    N = 1024  # parts x N = 2^20 > 2^19
    dB = torch.zeros((64, N), device="cuda")
    dC = torch.full((64, N), float("nan"), device="cuda")
    rows = torch.zeros(parts + 1, dtype=torch.int32, device="cuda")
    s = dA.struct()
    rc = fn(ctypes.byref(s), rows.data_ptr(), parts, dB.data_ptr(), dC.data_ptr(), N, None)
    assert rc == S.SPMM_UNSUPPORTED
    assert b"exceeds the carry workspace" in S.lib().spmm_c_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(dC).all()
