"""Device CSR -> BSR build and device fill-in statistics (additions; the
reference builds BSR on the host only, bsr.cu:30-109) against the host build,
which the oracle pins (test_oracle_pins / test_host_api).  The bar is bitwise
identity of row_ptr, col_idx and the fp16 bits of every stored element."""
import ctypes

import numpy as np
import pytest

from gpu_util import make_config

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _matrices(S):
    rng = np.random.default_rng(2024)
    out = {
        "uniform_small": S.generate_uniform_random_csr(300, 500, 0.03, 1),
        "ragged_dims": S.generate_uniform_random_csr(45, 70, 0.2, 2),
        "banded": S.generate_banded_csr(1000, 1000, 37, 3),
        "block_diag": S.generate_block_diagonal_csr(512, 600, 48, 4),
        "power_law": S.generate_power_law_csr(3000, 2500, 40.0, 1.5, 2500, 5),
        "empty_nnz": S.csr_from_coo_host(77, 33, [], [], []),
        "one_by_one": S.csr_from_coo_host(1, 1, [0], [0], [0.5]),
        "k_is_1": S.csr_from_coo_host(40, 1, np.arange(0, 40, 3), np.zeros(14, int),
                                      rng.uniform(-1, 1, 14)),
        "wide_k": S.csr_from_coo_host(64, 1_000_000, rng.integers(0, 64, 500),
                                      rng.integers(0, 1_000_000, 500), rng.uniform(-1, 1, 500)),
    }
    # repeated (row, col) cells: the last occurrence must be the stored one
    r = np.array([0, 0, 0, 5, 5, 17, 17, 17, 40])
    c = np.array([3, 3, 3, 9, 9, 100, 2, 100, 40])
    v = np.array([1.0, 2.0, 3.0, -1.0, -2.0, 7.0, 8.0, 9.0, 0.25])
    out["duplicates"] = S.csr_from_coo_host(48, 128, r, c, v)
    # values that exercise fp16 rounding: ties, overflow to inf, subnormals
    vals = np.array([1.0004883, 1.0014648, 65520.0, -70000.0, 3e-8, 6e-8, -1e-9, 0.1, 2049.0,
                     1e-5], np.float32)
    out["rounding"] = S.csr_from_coo_host(10, 16, np.arange(10), np.arange(10), vals)
    return out


def _equals_oracle(O, A, dev):
    """The device build is bitwise the oracle's restatement of bsr_from_csr_host
    (bsr.cu:30-109): block row pointers, ascending block-columns, RNE fp16."""
    brp, bci, bv = O.bsr_build(A.num_rows, A.num_cols, A.row_ptr, A.col_idx, A.values)
    assert np.array_equal(dev.row_ptr, brp)
    assert np.array_equal(dev.col_idx, bci)
    assert np.array_equal(dev.values, bv)


def _build_both(S, A):
    host = S.bsr_from_csr_host(A)
    built = S.bsr_from_csr_device(S.DeviceCSR(A))
    dev = built.to_host()
    return host, dev, built


@pytest.mark.parametrize("name", ["uniform_small", "ragged_dims", "banded", "block_diag",
                                  "power_law", "empty_nnz", "one_by_one", "k_is_1", "wide_k",
                                  "duplicates", "rounding"])
def test_device_build_equals_host(S, O, torch, name):
    A = _matrices(S)[name]
    say(f"bsr build case={name} M={A.num_rows} K={A.num_cols} nnz={A.nnz}")
    host, dev, built = _build_both(S, A)
    _equals_oracle(O, A, dev)
    assert (dev.num_rows, dev.num_cols, dev.block_rows, dev.block_cols, dev.nnz) == \
        (host.num_rows, host.num_cols, host.block_rows, host.block_cols, host.nnz)
    assert np.array_equal(dev.row_ptr, host.row_ptr)
    assert np.array_equal(dev.col_idx, host.col_idx)
    assert np.array_equal(dev.values, host.values)
    st_d = S.bsr_stats_from_csr_device(S.DeviceCSR(A))
    st_h = S.bsr_compute_stats(host)
    for f in ("num_blocks", "stored_elements", "original_nnz", "fill_in_ratio", "block_density"):
        assert getattr(st_d, f) == getattr(st_h, f), f


@pytest.mark.parametrize("cfg", ["c1", "c3", "c4", "c5"])
def test_device_build_configs_and_product(S, O, torch, cfg):
    A, B = make_config(S, cfg)
    say(f"bsr build config={cfg} nnz={A.nnz}")
    host, dev, built = _build_both(S, A)
    _equals_oracle(O, A, dev)
    assert np.array_equal(dev.row_ptr, host.row_ptr)
    assert np.array_equal(dev.col_idx, host.col_idx)
    assert np.array_equal(dev.values, host.values)
    # the MFMA product over the device-built BSR is the product over the host build
    B16 = S.float_to_half(torch.from_numpy(B).cuda())
    C_dev = S.spmm_wmma(built, B16)
    C_host = S.spmm_wmma(S.DeviceBSR(host), B16)
    torch.cuda.synchronize()
    assert torch.equal(C_dev, C_host)


def test_device_build_rejects_unsorted_rows(S, torch):
    A = S.HostCSR(2, 64, np.array([0, 3, 4], np.int32), np.array([5, 40, 7, 1], np.int32),
                  np.ones(4, np.float32))
    with pytest.raises(S.SpmmError) as e:
        S.bsr_from_csr_device(S.DeviceCSR(A))
    assert e.value.code == S.SPMM_UNSUPPORTED and "ascending" in str(e.value)
    # the hybrid's MFMA branch accepts it (it builds such input on the host)
    plan = S.hybrid_choose(A, 16, threshold=1000.0)
    assert plan.backend_name == "wmma"
    C, _ = S.hybrid_run(plan, A, np.ones((64, 16), np.float32), warmup=0, iters=1)
    assert np.allclose(C[0], 3.0) and np.allclose(C[1], 1.0)


def test_device_build_rejects_bad_columns(S, torch):
    A = S.HostCSR(2, 64, np.array([0, 1, 2], np.int32), np.array([5, 64], np.int32),
                  np.ones(2, np.float32))
    with pytest.raises(S.SpmmError) as e:
        S.bsr_from_csr_device(S.DeviceCSR(A))
    assert e.value.code == S.SPMM_INVALID
    wide = S.csr_from_coo_host(16, 4_128_769, [0], [4_128_768], [1.0])
    with pytest.raises(S.SpmmError) as e:
        S.bsr_stats_from_csr_device(S.DeviceCSR(wide))
    assert e.value.code == S.SPMM_UNSUPPORTED
    ok = S.csr_from_coo_host(16, 4_128_768, [0, 3], [0, 4_128_767], [1.0, 2.0])
    st = S.bsr_stats_from_csr_device(S.DeviceCSR(ok))
    assert st.num_blocks == 2


def test_device_build_null_arguments(S, torch):
    assert S.lib().spmm_c_bsr_from_csr_device(None, None, None) == S.SPMM_INVALID
