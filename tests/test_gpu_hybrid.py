"""Hybrid dispatch end to end on the GPU (spmm_hybrid.cu:32-125): the plan on
each BASELINE config, host-in/host-out execution of the chosen back end, and
the parity of its result."""
import numpy as np
import pytest

from gpu_util import CONFIGS, check_bsr, check_csr, make_config

pytestmark = pytest.mark.gpu

EXPECTED_BACKEND = {"c1": "csr", "c2": "csr", "c3": "wmma", "c4": "wmma", "c5": "csr"}


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_hybrid_plan_and_run(S, O, cfg):
    A, B = make_config(S, cfg)
    N = B.shape[1]
    plan = S.hybrid_choose(A, N)
    print(f"hybrid config={cfg} backend={plan.backend_name} fill={plan.fill_in_ratio:.4f}",
          flush=True)
    assert plan.backend_name == EXPECTED_BACKEND[cfg]
    C, ms = S.hybrid_run(plan, A, B, warmup=1, iters=3)
    assert ms > 0
    if plan.backend_name == "csr":
        C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
        check_csr(C, C64, absC)
    else:
        hb = S.bsr_from_csr_host(A)
        B16 = O.f32_to_f16(B)
        C32 = O.bsr_spmm_f32(A.num_rows, A.num_cols, hb.row_ptr, hb.col_idx, hb.values, B16,
                             threads=16)
        _, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values,
                                 B16.view(np.float16).astype(np.float32), threads=16)
        check_bsr(C, C32, absC)


def _batch_us(torch, launch, reps=50):
    """Best of three batches of `reps` back-to-back launches, in us per launch."""
    launch(5)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(3):
        e0.record()
        launch(reps)
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / reps * 1000.0)
    return best


def _csr_auto_launcher(S, torch, A, dB, dC):
    """The CSR form spmm_hybrid_run runs on A (spmm_hybrid.cu:103-116's role):
    row groups, the engine with the longest row as hint, merge-path, or
    merge-path over B-row halves."""
    form, opts, parts = S.csr_auto_form(A, int(dB.shape[1]))
    if form == "khalf":
        kp = S.KHalfPlan(A, int(dB.shape[1]))
        return form, lambda n: kp.launch_repeat(dB, dC, n)
    dA = S.DeviceCSR(A)
    if form == "split":
        rows = torch.from_numpy(S.nnz_split_rows(A, parts)).cuda()
        carry = torch.empty((parts, int(dB.shape[1])), device="cuda")
        return form, lambda n: S.launch_repeat_split(dA, rows, dB, dC, carry, n)
    return form, lambda n: S.launch_repeat_opts(dA, dB, dC, opts, n)


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_hybrid_picks_faster_backend(S, cfg):
    # The default plan names the faster back end on this GPU, each timed in
    # the form spmm_hybrid_run actually runs (CSR: csr_auto_form's choice).
    # Inside a 10% margin either choice is accepted (timing noise near the
    # crossover); outside it the plan must name the faster one.
    import torch
    A, B = make_config(S, cfg)
    N = B.shape[1]
    plan = S.hybrid_choose(A, N)
    dB = torch.from_numpy(B).cuda()
    dC = torch.empty((A.num_rows, N), device="cuda")
    form, csr_launch = _csr_auto_launcher(S, torch, A, dB, dC)
    t_csr = _batch_us(torch, csr_launch)
    dAb = S.DeviceBSR(S.bsr_from_csr_host(A))
    B16 = S.float_to_half(dB)
    try:  # the run-panel form on structured matrices, else the record kernel
        tile = S.BsrTilePlan(dAb)
        t_mma = _batch_us(torch, lambda n: tile.launch_repeat(B16, dC, n))
    except S.SpmmError as e:
        assert e.code == S.SPMM_UNSUPPORTED
        t_mma = _batch_us(torch, lambda n: S.launch_repeat("wmma", dAb, B16, dC, n))
    print(f"hybrid config={cfg} csr({form})_us={t_csr:.2f} wmma_us={t_mma:.2f} "
          f"plan={plan.backend_name}", flush=True)
    if max(t_csr, t_mma) <= 1.10 * min(t_csr, t_mma):
        return
    assert plan.backend_name == ("wmma" if t_mma < t_csr else "csr")


def test_hybrid_forced_backends_agree(S, O):
    # both back ends on the same fp16-exact input give the same product
    A, B = make_config(S, "c3")
    csr = S.hybrid_choose(A, B.shape[1], threshold=0.5)   # fill 1.1158 > 0.5 -> CSR
    mma = S.hybrid_choose(A, B.shape[1], threshold=2.0)
    assert csr.backend_name == "csr" and mma.backend_name == "wmma"
    C1, _ = S.hybrid_run(csr, A, B, warmup=0, iters=1)
    C2, _ = S.hybrid_run(mma, A, B, warmup=0, iters=1)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    check_csr(C1, C64, absC)
    check_csr(C2, C64, absC)


NARROW_CASES = {
    # (generator, N, expected back end): clear-cut cases of the per-N cut-off
    "banded_n32": (lambda S: S.generate_banded_csr(8192, 8192, 64, 1003), 32, "wmma"),
    "uniform_fill20_n16": (lambda S: S.generate_uniform_random_csr(8192, 8192, 0.05, 42), 16,
                           "csr"),
    "uniform_fill33_n32": (lambda S: S.generate_uniform_random_csr(8192, 8192, 0.03, 42), 32,
                           "csr"),
}


@pytest.mark.parametrize("case", sorted(NARROW_CASES))
def test_hybrid_narrow_b(S, O, case):
    # the per-N cut-off at narrow B: the plan names the back end that is
    # faster there (margins of 1.7x or more), runs it through spmm_hybrid_run
    # (row groups on the CSR side) and is faster than the forced other one
    gen, N, want = NARROW_CASES[case]
    A = gen(S)
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(np.random.default_rng(N).uniform(-1, 1, (A.num_cols, N))
                        .astype(np.float32))
    plan = S.hybrid_choose(A, N)
    other = S.hybrid_choose(A, N, threshold=(0.5 if want == "wmma" else 1e9))
    print(f"hybrid narrow case={case} N={N} fill={plan.fill_in_ratio:.2f} "
          f"threshold={plan.threshold} plan={plan.backend_name}", flush=True)
    assert plan.backend_name == want and other.backend_name != want
    C, ms = S.hybrid_run(plan, A, B, warmup=3, iters=30)
    _, ms_other = S.hybrid_run(other, A, B, warmup=3, iters=30)
    print(f"  ms={ms:.4f} other_ms={ms_other:.4f}", flush=True)
    assert ms < ms_other
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A.values, B, threads=16)
    if want == "csr":
        check_csr(C, C64, absC)
    else:
        check_csr(C, C64, absC, tol=1e-5)
