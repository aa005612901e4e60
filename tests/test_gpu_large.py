"""Large inputs on one MI355X: the engine at sizes far beyond the BASELINE
configs, where 32-bit offsets, grid limits and the 2 GiB structured-buffer
limit would show.  The oracle (fp64 loop, reference-independent) checks a
random sample of rows, and linearity in B checks the whole output:
C(A, B1 + B2) = C(A, B1) + C(A, B2) up to fp32 rounding.

* 1 M x 1 M CSR, 32 entries per row (33.5 M nonzeros), N = 256: B and C of
  1 GiB each, through the CSR form spmm_hybrid_run picks.
* 131 072 x 2 560 000 CSR with N = 256: B of 2.6 GB, past the 2 GiB a
  structured buffer can address, so the engine falls back to 64-bit address
  loads.
* banded 262 144^2 (half-bandwidth 32) on the MFMA path with N = 128, and the
  run-panel form on it and on block-diagonal 262 144^2 (1024 blocks of 256^2)
  at N = 256.
* 262 144 x 16 384 power-law rows (mean 164, capped at 4096; ~43 M nonzeros) with N = 128:
  B of 8 MiB, so the hybrid's form is merge-path over B-row halves.
"""
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


def _random_rows(S, M, K, per_row, seed):
    rng = np.random.default_rng(seed)
    cols = rng.integers(0, K, size=(M, per_row), dtype=np.int32)
    cols.sort(axis=1)
    vals = rng.uniform(-1, 1, size=M * per_row).astype(np.float32)
    row_ptr = np.arange(0, M * per_row + 1, per_row, dtype=np.int32)
    return S.HostCSR(M, K, row_ptr, cols.reshape(-1), vals)


def _sample_ref(A, B, rows):
    """fp64 rows of A*B and of |A||B| for the sampled rows."""
    ref = np.zeros((rows.size, B.shape[1]))
    absr = np.zeros_like(ref)
    for i, r in enumerate(rows):
        p0, p1 = A.row_ptr[r], A.row_ptr[r + 1]
        Bk = B[A.col_idx[p0:p1]].astype(np.float64)
        v = A.values[p0:p1].astype(np.float64)
        ref[i] = v @ Bk
        absr[i] = np.abs(v) @ np.abs(Bk)
    return ref, absr


def _csr_launch(S, torch, A, dA, dB, C):
    form, opts, parts = S.csr_auto_form(A, int(dB.shape[1]))
    stream = torch.cuda.current_stream()
    if form == "khalf":
        S.KHalfPlan(A, int(dB.shape[1])).launch_repeat(dB, C, 1, stream)
    elif form == "split":
        rows = torch.from_numpy(S.nnz_split_rows(A, parts)).cuda()
        carry = torch.empty((parts, dB.shape[1]), dtype=torch.float32, device="cuda")
        S.launch_repeat_split(dA, rows, dB, C, carry, 1, stream)
    else:
        S.launch_repeat_opts(dA, dB, C, opts, 1, stream)
    return form


@pytest.mark.parametrize("shape", ["uniform_1m_n256", "b_past_2gib"])
def test_large_csr(S, torch, shape):
    if shape == "uniform_1m_n256":
        M, K, per_row, N, seed = 1 << 20, 1 << 20, 32, 256, 71
    else:
        M, K, per_row, N, seed = 131072, 2_560_000, 16, 256, 72
    A = _random_rows(S, M, K, per_row, seed)
    rng = np.random.default_rng(seed + 1)
    B1 = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
    say(f"large csr shape={shape} M={M} K={K} nnz={A.nnz} N={N} "
        f"B bytes={B1.nbytes} C bytes={M * N * 4}")
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B1).cuda()
    C1 = torch.full((M, N), float("nan"), device="cuda")
    form = _csr_launch(S, torch, A, dA, dB, C1)
    torch.cuda.synchronize()
    say(f"large csr shape={shape} form={form}")
    rows = np.sort(rng.choice(M, size=2000, replace=False))
    ref, absr = _sample_ref(A, B1, rows)
    got = C1[torch.from_numpy(rows).cuda()].cpu().numpy()
    check_csr(got, ref, absr)
    assert not torch.isnan(C1).any().item(), "every row of C is written"
    # linearity over the whole output: A(B1 + B2) = A B1 + A B2
    B2 = torch.empty_like(dB).uniform_(-1, 1, generator=torch.Generator("cuda").manual_seed(seed))
    C2 = torch.empty_like(C1)
    _csr_launch(S, torch, A, dA, B2, C2)
    B12 = dB + B2
    del dB
    C12 = torch.empty_like(C1)
    _csr_launch(S, torch, A, dA, B12, C12)
    torch.cuda.synchronize()
    diff = (C12 - (C1 + C2)).abs().max().item()
    scale = C12.abs().max().item()
    assert diff <= 1e-5 * max(scale, 1.0) * per_row, (diff, scale)


def test_large_mfma(S, O, torch):
    M = 262144
    A = S.generate_banded_csr(M, M, 32, 73)
    A.values = S.round_to_fp16(A.values)
    rng = np.random.default_rng(74)
    B = S.round_to_fp16(rng.uniform(-1, 1, size=(M, 128)).astype(np.float32))
    hb = S.bsr_from_csr_host(A)
    say(f"large mfma banded M={M} nnz={A.nnz} blocks={hb.num_blocks} N=128")
    B16 = O.f32_to_f16(B)
    C = S.spmm_wmma(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda())
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(M, size=2000, replace=False))
    Bh = B16.view(np.float16).astype(np.float32)
    ref, absr = _sample_ref(A, Bh, rows)
    got = C[torch.from_numpy(rows).cuda()].cpu().numpy()
    check_bsr(got, ref, absr)
    check_csr(got, ref, absr, tol=1e-5)  # fp16 products are exact in fp32
    assert not torch.isnan(C).any().item()


@pytest.mark.parametrize("kind", ["band", "diag"])
def test_large_tile(S, O, torch, kind):
    # The run-panel form at 262144 rows (the hybrid's MFMA form on structured
    # input): sampled rows against fp64, every row written, and whole-output
    # sign symmetry (within rounding) and determinism through the same plan.
    M = 262144
    if kind == "band":
        A, N = S.generate_banded_csr(M, M, 32, 76), 128
    else:
        A, N = S.generate_block_diagonal_csr(M, M, 256, 77, 0.1), 256
    A.values = S.round_to_fp16(A.values)
    rng = np.random.default_rng(78)
    B = S.round_to_fp16(rng.uniform(-1, 1, size=(M, N)).astype(np.float32))
    hb = S.bsr_from_csr_host(A)
    dA = S.DeviceBSR(hb)
    plan = S.BsrTilePlan(dA)
    say(f"large tile {kind} M={M} nnz={A.nnz} blocks={hb.num_blocks} N={N} "
        f"panels={plan.panels} max_union={plan.max_union} shape={plan.default_shape(N)}")
    B16 = O.f32_to_f16(B)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    C1 = torch.full((M, N), float("nan"), device="cuda")
    plan.launch(dB, C1)
    torch.cuda.synchronize()
    assert not torch.isnan(C1).any().item(), "every row of C is written"
    rows = np.sort(rng.choice(M, size=2000, replace=False))
    Bh = B16.view(np.float16).astype(np.float32)
    ref, absr = _sample_ref(A, Bh, rows)
    got = C1[torch.from_numpy(rows).cuda()].cpu().numpy()
    check_bsr(got, ref, absr)
    check_csr(got, ref, absr, tol=1e-5)  # fp16 products are exact in fp32
    # whole output: C(A, -B) = -C(A, B) within fp32 rounding (the matrix cores'
    # internal accumulation is not sign-symmetric to the last bit), and a
    # second launch reproduces C bit for bit
    Cneg = plan.launch((-dB.view(torch.float16)).contiguous().view(torch.int16))
    Cagain = plan.launch(dB)
    torch.cuda.synchronize()
    asym = (Cneg + C1).abs()
    say(f"large tile {kind}: C(-B) + C(B) max {asym.max().item():.3e} over "
        f"{int((asym > 0).sum().item())} of {asym.numel()} elements; max |C| "
        f"{C1.abs().max().item():.3f}")
    assert asym.max().item() <= 1e-5 * C1.abs().max().item()
    assert torch.equal(Cagain, C1)
    plan.close()


def test_large_khalf(S, torch):
    M, K, N, seed = 262144, 16384, 128, 75
    A = S.generate_power_law_csr(M, K, 164.0, 1.5, 4096, seed)
    assert S.csr_auto_form(A, N)[0] == "khalf"
    rng = np.random.default_rng(seed + 1)
    B1 = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
    say(f"large khalf M={M} K={K} nnz={A.nnz} N={N}")
    with S.KHalfPlan(A, N) as p:
        dB = torch.from_numpy(B1).cuda()
        C1 = torch.full((M, N), float("nan"), device="cuda")
        p.launch(dB, C1)
        torch.cuda.synchronize()
        rows = np.sort(rng.choice(M, size=2000, replace=False))
        ref, absr = _sample_ref(A, B1, rows)
        check_csr(C1[torch.from_numpy(rows).cuda()].cpu().numpy(), ref, absr)
        assert not torch.isnan(C1).any().item(), "every row of C is written"
        # linearity over the whole output through the same plan
        B2 = torch.empty_like(dB).uniform_(-1, 1, generator=torch.Generator("cuda").manual_seed(seed))
        C2 = torch.empty_like(C1)
        p.launch(B2, C2)
        C12 = torch.empty_like(C1)
        p.launch(dB + B2, C12)
        torch.cuda.synchronize()
        diff = (C12 - (C1 + C2)).abs().max().item()
        scale = C12.abs().max().item()
        assert diff <= 1e-5 * max(scale, 1.0) * 64, (diff, scale)
