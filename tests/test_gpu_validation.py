"""The Python binding rejects malformed device operands before any launch.

The C ABI takes bare pointers and sizes (spmm_tiled_v3.h:40, spmm_wmma.h:39
take `const float* d_B, float* d_C, int N`), so a transposed B, a short C or
an fp32 tensor passed as fp16 would read or write out of bounds on the device.
Every wrapper validates with one helper and raises SpmmError(SPMM_INVALID);
C keeps its NaN fill, so no kernel ran.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")


class _FakeA:
    """Just the fields the validation reads (num_rows, num_cols, row_ptr)."""

    def __init__(self, rows, cols):
        self.num_rows, self.num_cols = rows, cols
        self.row_ptr = torch.zeros(rows + 1, dtype=torch.int32)


def test_cpu_tensors_rejected(S):
    A = _FakeA(4, 4)
    with pytest.raises(S.SpmmError) as e:
        S.spmm_csr("tiled_v3", A, torch.zeros(4, 8))
    assert e.value.code == S.SPMM_INVALID and "cuda" in str(e.value)
    with pytest.raises(S.SpmmError):
        S.spmm_wmma(A, np.zeros((4, 8), np.int16))


def test_host_b_shape_rejected(S):
    A = S.generate_uniform_random_csr(32, 24, 0.2, 1)
    with pytest.raises(S.SpmmError) as e:
        S.hybrid_run(S.hybrid_choose(A, 16), A, np.zeros((23, 16), np.float32))
    assert e.value.code == S.SPMM_INVALID
    with pytest.raises(S.SpmmError):
        S.hybrid_run(S.hybrid_choose(A, 16), A, np.zeros(24 * 16, np.float32))


@pytest.fixture(scope="module")
def dev(S):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    A = S.generate_uniform_random_csr(64, 48, 0.1, 7)
    B = torch.from_numpy(S.generate_dense_row_major(48, 32, 8)).cuda()
    return S.DeviceCSR(A), B


def _nan_c(rows, cols):
    return torch.full((rows, cols), float("nan"), dtype=torch.float32, device="cuda")


def _rejects(S, fn, C=None):
    with pytest.raises(S.SpmmError) as e:
        fn()
    assert e.value.code == S.SPMM_INVALID, e.value
    if C is not None:
        torch.cuda.synchronize()
        assert torch.isnan(C).all(), "a kernel wrote C before the operands were checked"


@pytest.mark.gpu
def test_csr_operands_rejected(S, dev):
    dA, B = dev
    C = _nan_c(64, 32)
    Bt = torch.from_numpy(S.generate_dense_row_major(32, 48, 9)).cuda().t()  # 48 x 32 view
    assert not Bt.is_contiguous()
    for k in ("baseline", "tiled_v3", "tiled_v4"):
        _rejects(S, lambda: S.spmm_csr(k, dA, Bt, C), C)                       # transposed B
    _rejects(S, lambda: S.spmm_csr("tiled_v3", dA, B[:47], C), C)             # K mismatch
    _rejects(S, lambda: S.spmm_csr("tiled_v3", dA, B.double(), C), C)         # dtype
    _rejects(S, lambda: S.spmm_csr("tiled_v3", dA, B, _nan_c(63, 32)))        # C too short
    _rejects(S, lambda: S.spmm_csr("tiled_v3", dA, B, _nan_c(64, 31)))        # C too narrow
    _rejects(S, lambda: S.spmm_csr("tiled_v3", dA, B, C.half()))              # C dtype
    _rejects(S, lambda: S.spmm_csr("tiled_v3", dA, B.cpu(), C), C)            # host B
    _rejects(S, lambda: S.spmm_tiled_v3_opts(dA, Bt, S.EngineOptsT(), C), C)
    _rejects(S, lambda: S.launch_repeat("tiled_v3", dA, Bt, C, 3), C)
    _rejects(S, lambda: S.launch_repeat_opts(dA, B, _nan_c(64, 16), S.EngineOptsT(), 3))
    _rejects(S, lambda: S.time_repeat("tiled_v3", dA, B[:, :16], C, 3), C)   # strided view


@pytest.mark.gpu
def test_partition_operands_rejected(S, dev):
    dA, B = dev
    C = _nan_c(64, 32)
    rows = torch.tensor([0, 32, 64], dtype=torch.int32, device="cuda")
    _rejects(S, lambda: S.spmm_tiled_v3_partitioned(dA, rows.long(), B, C), C)
    _rejects(S, lambda: S.spmm_tiled_v3_partitioned(dA, rows[:1], B, C), C)
    split = torch.tensor([0, 10, 63], dtype=torch.int32, device="cuda")
    short = torch.empty(2 * 32 - 1, dtype=torch.float32, device="cuda")
    _rejects(S, lambda: S.spmm_tiled_v3_split(dA, split, B, C, carry=short), C)
    _rejects(S, lambda: S.spmm_tiled_v3_split(dA, split.float(), B, C), C)
    _rejects(S, lambda: S.launch_repeat_split(dA, split, B, C, None, 2), C)


@pytest.mark.gpu
def test_bsr_operands_rejected(S):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    A = S.generate_banded_csr(64, 64, 5, 3)
    dA = S.DeviceBSR(S.bsr_from_csr_host(A))
    B32 = torch.from_numpy(S.generate_dense_row_major(64, 32, 4)).cuda()
    B16 = B32.half()
    C = _nan_c(64, 32)
    _rejects(S, lambda: S.spmm_wmma(dA, B32, C), C)                           # fp32 as fp16
    _rejects(S, lambda: S.spmm_wmma(dA, B16[:63], C), C)                      # K mismatch
    _rejects(S, lambda: S.spmm_wmma(dA, B16, _nan_c(64, 16)))                 # C narrow
    _rejects(S, lambda: S.spmm_wmma_opts(dA, B16.t(), S.BsrOptsT(), C), C)   # non-contiguous
    _rejects(S, lambda: S.launch_repeat_wmma_opts(dA, B16, C[:32], S.BsrOptsT(), 2), C)
    _rejects(S, lambda: S.launch_repeat("wmma", dA, B32, C, 2), C)
    # option values no kernel has, values the named kernel lacks (panel depth
    # 3, panel tiles 2, wave tiles 8) and nonzero reserved slots
    for opts in (S.BsrOptsT(4, 4, 0, 3), S.BsrOptsT(8, 2, 0, 2), S.BsrOptsT(1, 8, 0, 2),
                 S.BsrOptsT(0, 0, 0, 8), S.BsrOptsT(reserved0=1), S.BsrOptsT(reserved1=4)):
        _rejects(S, lambda: S.spmm_wmma_opts(dA, B16, opts, C), C)
    # a correct call still works
    S.spmm_wmma(dA, B16, C)
    torch.cuda.synchronize()
    assert not torch.isnan(C).any()


@pytest.mark.gpu
def test_float_to_half_operands_rejected(S):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    src = torch.linspace(-1, 1, 1000, device="cuda")
    dst = torch.full((999,), float("nan"), dtype=torch.float16, device="cuda")
    _rejects(S, lambda: S.float_to_half(src.double()))
    _rejects(S, lambda: S.float_to_half(src.to(torch.int32)))
    _rejects(S, lambda: S.float_to_half(src, dst))                            # 999 < 1000
    _rejects(S, lambda: S.float_to_half(src, torch.empty(1000, device="cuda")))  # fp32 dst
    _rejects(S, lambda: S.float_to_half(src.reshape(20, 50).t()))             # non-contiguous
    torch.cuda.synchronize()
    assert torch.isnan(dst).all()
    out = S.float_to_half(src)
    torch.cuda.synchronize()
    assert torch.equal(out, src.half())
