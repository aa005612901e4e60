"""Unified-memory path on one GPU (role of spmm_unified, spmm_multigpu.cu:122-182)
against the fp64 oracle, through the C ABI."""
import numpy as np
import pytest

from gpu_util import check_csr, make_config

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _residency(S):
    """How the unified path placed A, B and C on this device: 1 managed and
    prefetched, 0 managed but moved on first touch, -1 no managed memory on the
    device (device allocations filled by explicit copies)."""
    A = S.csr_from_coo_host(16, 16, [0], [0], [1.0])
    C, ms, res = S.unified_run(A, np.ones((16, 16), np.float32), warmup=0, iters=1)
    assert res in (-1, 0, 1) and ms >= 0
    assert C[0, 0] == 1.0 and not C[1:].any()
    return res


def test_gpu_count(S):
    assert S.gpu_count() >= 1


def test_unified_contract(S):
    # a working path on every device: managed memory where the device has it,
    # device copies where it does not (no fault, no exit)
    say(f"unified residency on this device: {_residency(S)}")


@pytest.mark.parametrize("case", ["c1", "ragged", "empty"])
def test_unified_matches_oracle(S, O, case):
    if case == "c1":
        A, B = make_config(S, "c1")
    elif case == "ragged":
        rng = np.random.default_rng(8)
        A = S.generate_power_law_csr(700, 900, 30.0, 1.5, 900, 9)
        B = rng.uniform(-1, 1, (900, 96)).astype(np.float32)
    else:
        A = S.csr_from_coo_host(40, 30, [], [], [])
        B = np.ones((30, 64), np.float32)
    say(f"unified case={case} M={A.num_rows} nnz={A.nnz} N={B.shape[1]}")
    C, ms, res = S.unified_run(A, B, warmup=1, iters=3)
    say(f"  ms={ms:.4f} residency={res}")
    assert res in (-1, 0, 1)
    assert ms >= 0
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    check_csr(C, C64, absC)
