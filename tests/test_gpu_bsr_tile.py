"""GPU parity of the run-panel form of spmm_wmma (bsr_tile.hip: the MFMA form
spmm_hybrid_run runs on structured matrices) against the oracle, through the
C ABI on cuda:0.

Bar (north star): within 1e-2 relative of fp32 accumulation of the same
fp16-rounded operands (gpu_util.check_bsr), and the tight check against the
exact fp64 product of the fp16 operands (fp16 products are exact in fp32, so
only fp32 summation error remains: 1e-5 of |A16||B16|), which catches operand
layout, swizzle and pairing mistakes.  Every kernel shape runs on every case
its union fits: banded and block-diagonal matrices with odd sizes, empty
block-rows, runs starting on odd slots, odd run lengths (the 16x16x16 tail),
narrow and wide N, and unions wider than the one-shot forms hold (the ring).
"""
import numpy as np
import pytest

from gpu_util import check_bsr, check_csr
from spmm_amd import SPMM_INVALID, SPMM_UNSUPPORTED

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _refs(S, O, A, B):
    hb = S.bsr_from_csr_host(A)
    B16 = O.f32_to_f16(B)
    C32 = O.bsr_spmm_f32(A.num_rows, A.num_cols, hb.row_ptr, hb.col_idx, hb.values, B16, threads=16)
    A16 = A.values.astype(np.float16).astype(np.float32)
    Bh = B16.view(np.float16).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A16, Bh, threads=16)
    return hb, B16, C32, C64, absC


def _case(S, kind, M, K, param, N, seed):
    A = (S.generate_banded_csr(M, K, param, seed) if kind == "band"
         else S.generate_block_diagonal_csr(M, K, param, seed, 0.1))
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(np.random.default_rng(seed).uniform(-1, 1, (K, N)).astype(np.float32))
    return A, B


CASES = [
    # kind, M, K, param (half-bandwidth / diagonal block), N
    ("band", 1000, 1000, 20, 136),   # odd sizes, runs starting on odd slots, odd lengths
    ("band", 512, 512, 64, 64),      # c3's band on a small matrix
    ("band", 300, 200, 0, 8),        # diagonal only: one-block runs, narrow N, ragged K
    ("band", 160, 160, 1, 40),
    ("diag", 512, 512, 256, 256),    # c4's blocks
    ("diag", 1000, 1000, 40, 24),    # diagonal blocks straddling block-rows
    ("diag", 400, 400, 48, 320),     # wide N
    ("diag", 1024, 1024, 512, 32),   # unions of 32 block-columns: the ring only
    ("diag", 1000, 1000, 128, 72),   # a partial last panel
]


@pytest.mark.parametrize("kind,M,K,param,N", CASES)
def test_tile_shapes(S, O, torch, kind, M, K, param, N):
    A, B = _case(S, kind, M, K, param, N, 7)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    dA = S.DeviceBSR(hb)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    shapes = S.bsr_tile_shapes()
    ran = 0
    for R in (4, 8):
        plan = S.BsrTilePlan(dA, R)
        for sid, sh in enumerate(shapes):
            if sh["R"] != R:
                continue
            dC = torch.full((M, N), float("nan"), device="cuda")
            if sh["KIND"] != 0 and sh["NB"] * sh["CS"] < plan.max_union:
                with pytest.raises(S.SpmmError) as e:
                    plan.launch(dB, dC, shape=sid)
                assert e.value.code == SPMM_INVALID
                continue
            say(f"tile case={kind} M={M} N={N} param={param} R={R} shape={sid} {sh} "
                f"max_union={plan.max_union}")
            plan.launch(dB, dC, shape=sid)
            torch.cuda.synchronize()
            C = dC.cpu().numpy()
            check_bsr(C, C32, absC)
            check_csr(C, C64, absC, tol=1e-5)
            ran += 1
        plan.close()
    assert ran >= 3


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_tile_full_configs(S, O, torch, name):
    # The BASELINE configs the hybrid runs in this form: the default shape and
    # one shape of each kind, against the oracle.
    from gpu_util import make_config
    A, B = make_config(S, name)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    dA = S.DeviceBSR(hb)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    plan = S.BsrTilePlan(dA)
    N = B.shape[1]
    default = plan.default_shape(N)
    shapes = S.bsr_tile_shapes()
    assert shapes[default]["KIND"] in (2, 3)  # the union fits a producer/consumer form
    picks = [-1] + [next(i for i, s in enumerate(shapes)
                         if s["KIND"] == k and s["R"] == 4
                         and (k == 0 or s["NB"] * s["CS"] >= plan.max_union))
                    for k in (0, 1, 2, 3)]
    for sid in picks:
        say(f"tile full config={name} shape={sid} default={default} max_union={plan.max_union}")
        C = plan.launch(dB, shape=sid)
        torch.cuda.synchronize()
        C = C.cpu().numpy()
        check_bsr(C, C32, absC)
        check_csr(C, C64, absC, tol=1e-5)


@pytest.mark.parametrize("seed", [77, 78, 79])
def test_tile_fuzz(S, O, torch, seed):
    # Seeded random run structures (tile_cases.random_case: random run starts
    # and lengths, empty block-rows, ragged M and K) at random N (multiples of 8),
    # every kernel shape whose union fits, R = 4 and 8, against the oracle.
    from tile_cases import random_case, panels_contiguous
    rng = np.random.default_rng(seed)
    shapes = S.bsr_tile_shapes()
    done = 0
    while done < 24:
        A, runs, M, K = random_case(S, rng)
        Rs = [R for R in (4, 8) if panels_contiguous(runs, R)]
        if not Rs:
            continue
        N = 8 * int(rng.integers(1, 34))
        B = S.round_to_fp16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
        hb, B16, C32, C64, absC = _refs(S, O, A, B)
        dA = S.DeviceBSR(hb)
        dB = torch.from_numpy(B16.view(np.int16)).cuda()
        for R in Rs:
            plan = S.BsrTilePlan(dA, R)
            for sid, sh in enumerate(shapes):
                if sh["R"] != R or (sh["KIND"] != 0 and sh["NB"] * sh["CS"] < plan.max_union):
                    continue
                say(f"tile fuzz case={done} M={M} K={K} N={N} blocks={hb.num_blocks} R={R} "
                    f"shape={sid} max_union={plan.max_union}")
                dC = torch.full((M, N), float("nan"), device="cuda")
                plan.launch(dB, dC, shape=sid)
                torch.cuda.synchronize()
                C = dC.cpu().numpy()
                check_bsr(C, C32, absC)
                check_csr(C, C64, absC, tol=1e-5)
            plan.close()
        done += 1


def test_tile_matches_wmma(S, O, torch):
    # Same products, same sums: within fp32 rounding of the record kernel.
    A, B = _case(S, "band", 512, 512, 30, 128, 11)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    dA = S.DeviceBSR(hb)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    Cw = S.spmm_wmma(dA, dB).cpu().numpy().astype(np.float64)
    Ct = S.BsrTilePlan(dA).launch(dB).cpu().numpy().astype(np.float64)
    assert np.all(np.abs(Ct - Cw) <= 1e-5 * absC + 1e-30)


def test_tile_refusals(S, O, torch):
    # not runs -> the plan is refused; N % 8 != 0 -> the launch is refused;
    # a plan used with another matrix -> refused
    hb = S.bsr_from_csr_host(S.generate_uniform_random_csr(256, 256, 0.02, 3))
    with pytest.raises(S.SpmmError) as e:
        S.BsrTilePlan(S.DeviceBSR(hb))
    assert e.value.code == SPMM_UNSUPPORTED
    A, B = _case(S, "band", 256, 256, 16, 20, 4)
    hb = S.bsr_from_csr_host(A)
    dA = S.DeviceBSR(hb)
    plan = S.BsrTilePlan(dA)
    dB = torch.zeros((256, 20), dtype=torch.int16, device="cuda")
    with pytest.raises(S.SpmmError) as e:
        plan.launch(dB)
    assert e.value.code == SPMM_UNSUPPORTED
    other = S.DeviceBSR(S.bsr_from_csr_host(S.generate_banded_csr(128, 128, 16, 4)))
    plan.A = other
    with pytest.raises(S.SpmmError) as e:
        plan.launch(torch.zeros((128, 16), dtype=torch.int16, device="cuda"))
    assert e.value.code == SPMM_INVALID
    # the same matrix uploaded again: same sizes, other structure arrays -> refused
    plan.A = S.DeviceBSR(hb)
    with pytest.raises(S.SpmmError) as e:
        plan.launch(torch.zeros((256, 16), dtype=torch.int16, device="cuda"))
    assert e.value.code == SPMM_INVALID


def test_tile_empty_matrix(S, O, torch):
    # all-zero matrix: every panel's union is empty and C is all zeros
    A = S.csr_from_coo_host(96, 64, [], [], [])
    hb = S.bsr_from_csr_host(A)
    dA = S.DeviceBSR(hb)
    plan = S.BsrTilePlan(dA)
    assert plan.max_union == 0
    dB = torch.ones((64, 32), dtype=torch.int16, device="cuda")
    for sid, sh in enumerate(S.bsr_tile_shapes()):
        if sh["R"] != 4:
            continue
        dC = torch.full((96, 32), float("nan"), device="cuda")
        plan.launch(dB, dC, shape=sid)
        torch.cuda.synchronize()
        assert torch.count_nonzero(dC).item() == 0, sid
