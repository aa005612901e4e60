"""GPU parity of the BSR / matrix-core path (roles of spmm_wmma.cu) and of the
fp32 -> fp16 conversion, against the oracle, through the C ABI on cuda:0.

Bar (north star): within 1e-2 relative of fp32 accumulation of the same
fp16-rounded inputs (gpu_util.check_bsr).  A second, much tighter check
against the exact (fp64) product of the fp16 operands catches operand-layout
mistakes that a loose bar could hide.
"""
import numpy as np
import pytest

from gpu_util import check_bsr, check_csr, make_config

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need cuda:0"
    return t


def _refs(S, O, A, B):
    """(host BSR, fp16 bits of B, oracle fp32 result, fp64 exact, |A16||B16|)."""
    hb = S.bsr_from_csr_host(A)
    B16 = O.f32_to_f16(B)
    C32 = O.bsr_spmm_f32(A.num_rows, A.num_cols, hb.row_ptr, hb.col_idx, hb.values, B16, threads=16)
    A16 = A.values.astype(np.float16).astype(np.float32)
    Bh = B16.view(np.float16).astype(np.float32)
    C64, absC = O.csr_spmm_f64(A.row_ptr, A.col_idx, A16, Bh, threads=16)
    return hb, B16, C32, C64, absC


def _run_wmma(S, torch, hb, B16):
    dA = S.DeviceBSR(hb)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    dC = torch.full((hb.num_rows, B16.shape[1]), float("nan"), device="cuda")
    S.spmm_wmma(dA, dB, dC)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


def _no_duplicates(A):
    for r in range(A.num_rows):
        row = A.col_idx[A.row_ptr[r]:A.row_ptr[r + 1]]
        if np.unique(row).size != row.size:
            return False
    return True


def _cases(S):
    rng = np.random.default_rng(99)
    out = {}
    out["single_block"] = (S.csr_from_coo_host(16, 16, np.repeat(np.arange(16), 16),
                                                np.tile(np.arange(16), 16),
                                                rng.uniform(-1, 1, 256)),
                           rng.uniform(-1, 1, (16, 16)))
    out["odd_pair_count"] = (S.generate_banded_csr(48, 48, 1, 5), rng.uniform(-1, 1, (48, 32)))
    out["ragged_dims"] = (S.generate_uniform_random_csr(45, 70, 0.08, 6),
                          rng.uniform(-1, 1, (70, 48)))
    out["n_not_16"] = (S.generate_uniform_random_csr(64, 64, 0.1, 7), rng.uniform(-1, 1, (64, 20)))
    out["n_1"] = (S.generate_uniform_random_csr(64, 40, 0.1, 8), rng.uniform(-1, 1, (40, 1)))
    out["empty_block_rows"] = (S.csr_from_coo_host(80, 64, [0, 1, 70], [3, 60, 33], [1, 2, 3]),
                               rng.uniform(-1, 1, (64, 64)))
    out["empty"] = (S.csr_from_coo_host(33, 20, [], [], []), rng.uniform(-1, 1, (20, 16)))
    out["wide_n"] = (S.generate_banded_csr(256, 256, 20, 9), rng.uniform(-1, 1, (256, 320)))
    out["block_diag_small"] = (S.generate_block_diagonal_csr(512, 512, 64, 10),
                               rng.uniform(-1, 1, (512, 256)))
    for k, (A, B) in out.items():
        A.values = S.round_to_fp16(A.values)
        out[k] = (A, S.round_to_fp16(np.asarray(B, np.float32)))
    return out


@pytest.mark.parametrize("name", ["single_block", "odd_pair_count", "ragged_dims", "n_not_16",
                                  "n_1", "empty_block_rows", "empty", "wide_n",
                                  "block_diag_small"])
def test_wmma_cases(S, O, torch, name):
    A, B = _cases(S)[name]
    assert _no_duplicates(A)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    say(f"wmma case={name} M={A.num_rows} K={A.num_cols} N={B.shape[1]} blocks={hb.num_blocks}")
    C = _run_wmma(S, torch, hb, B16)
    check_bsr(C, C32, absC)
    # fp16 products are exact in fp32: only fp32 summation error remains
    check_csr(C, C64, absC, tol=1e-5)


def _variants():
    """(row_group, tiles, per_wave, depth, addressing) combinations that apply:
    the wave kernel (row_group 1, or per_wave) with 1/2/4 tiles per wave, 1/2/4
    pairs in flight and both addressings; the shared-panel kernel with 4 or 8
    block-rows per workgroup, 4 or 8 tiles per workgroup, 2 or 4 stages."""
    out = []
    for tiles in (1, 2, 4):
        for depth in (1, 2, 4):
            for addressing in (0, 1):
                out.append((1, tiles, 0, depth, addressing))
                out.append((0, tiles, 1, depth, addressing))
    for rg in (4, 8):
        for tiles in (4, 8):
            for depth in (2, 4):
                out.append((rg, tiles, 0, depth, 0))
    return out


@pytest.mark.parametrize("row_group,tiles,per_wave,depth,addressing", _variants())
def test_wmma_variants(S, O, torch, row_group, tiles, per_wave, depth, addressing):
    cases = _cases(S)
    for name in ("single_block", "odd_pair_count", "ragged_dims", "n_not_16", "n_1",
                 "empty_block_rows", "empty", "wide_n", "block_diag_small"):
        A, B = cases[name]
        hb, B16, C32, C64, absC = _refs(S, O, A, B)
        say(f"wmma opts row_group={row_group} tiles={tiles} per_wave={per_wave} depth={depth} "
            f"addressing={addressing} case={name}")
        dA = S.DeviceBSR(hb)
        dB = torch.from_numpy(B16.view(np.int16)).cuda()
        dC = torch.full((hb.num_rows, B16.shape[1]), float("nan"), device="cuda")
        S.spmm_wmma_opts(dA, dB, S.BsrOptsT(row_group, tiles, per_wave, depth, 0,
                                             addressing=addressing), dC)
        torch.cuda.synchronize()
        C = dC.cpu().numpy()
        check_bsr(C, C32, absC)
        check_csr(C, C64, absC, tol=1e-5)


def test_wmma_long_block_rows(S, O, torch):
    # block-rows with more than 64 blocks (the wave kernel's register chunk);
    # for the panel kernel a union wider than one pass of 126 slots
    A = S.generate_uniform_random_csr(64, 2048, 0.05, 31)
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(np.random.default_rng(3).uniform(-1, 1, (2048, 64)).astype(np.float32))
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    assert np.diff(hb.row_ptr).max() > 126  # so some panel's union takes two passes
    for rg, tiles, depth in ((4, 4, 2), (4, 8, 4), (8, 4, 4), (8, 8, 4), (1, 1, 0), (1, 2, 0),
                             (1, 4, 4)):
        say(f"wmma long block-rows row_group={rg} tiles={tiles} depth={depth} "
            f"blocks={hb.num_blocks}")
        C = S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(),
                             S.BsrOptsT(rg, tiles, 0, depth)).cpu().numpy()
        check_bsr(C, C32, absC)
        check_csr(C, C64, absC, tol=1e-5)


def test_wmma_chunk_boundaries(S, O, torch):
    # block-rows of exactly 63, 64, 65, 128 and 129 blocks: the wave kernel
    # reads block-columns 64 at a time and multiplies them in pairs
    rows, cols = [], []
    for br, nb in enumerate((63, 64, 65, 128, 129, 1, 0, 2)):
        for b in range(nb):
            rows.append(br * 16 + (b % 16))
            cols.append(b * 16 + (br % 16))
    A = S.csr_from_coo_host(8 * 16, 130 * 16, np.array(rows), np.array(cols),
                            np.random.default_rng(5).uniform(-1, 1, len(rows)).astype(np.float32))
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(np.random.default_rng(6).uniform(-1, 1, (130 * 16, 48)).astype(np.float32))
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    assert list(np.diff(hb.row_ptr)) == [63, 64, 65, 128, 129, 1, 0, 2]
    for tiles in (1, 2, 4):
        for depth in (1, 2, 4):
            for addressing in (0, 1):
                say(f"wmma chunk boundaries tiles={tiles} depth={depth} addressing={addressing}")
                C = S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(),
                                     S.BsrOptsT(1, tiles, 0, depth, 0,
                                                addressing=addressing)).cpu().numpy()
                check_bsr(C, C32, absC)
                check_csr(C, C64, absC, tol=1e-5)


def _dev_bsr(S, torch, M, K, row_ptr, col_idx, values16):
    """A device BSR from raw arrays (block-columns in any order, repeats allowed)."""
    hb = S.HostBSR(M, K, (M + 15) // 16, (K + 15) // 16, 0, np.asarray(row_ptr, np.int32),
                   np.asarray(col_idx, np.int32), np.asarray(values16, np.uint16))
    return hb, S.DeviceBSR(hb)


@pytest.mark.parametrize("order", ["descending", "repeated", "out_of_range"])
def test_panel_identity_union(S, O, torch, order):
    # Block-column lists that are not strictly ascending (or name block-columns
    # outside the matrix) take the panel kernel's identity union; the result
    # is the plain sum over the stored blocks either way.
    rng = np.random.default_rng(11)
    M, K, N = 80, 96, 64
    br, bc = (M + 15) // 16, (K + 15) // 16
    lists = [list(rng.choice(bc, int(rng.integers(1, bc + 1)), replace=False)) for _ in range(br)]
    if order == "descending":
        lists = [sorted(l, reverse=True) for l in lists]
    elif order == "repeated":
        lists = [sorted(l + l[:2]) for l in lists]
    else:
        lists = [sorted(l) + [bc + 3] for l in lists]
    row_ptr = np.concatenate([[0], np.cumsum([len(l) for l in lists])])
    col_idx = np.concatenate(lists)
    vals = O.f32_to_f16(rng.uniform(-1, 1, len(col_idx) * 256).astype(np.float32))
    B = S.round_to_fp16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    B16 = O.f32_to_f16(B)
    # dense reference: stored blocks summed (columns beyond K contribute nothing)
    Ad = np.zeros((br * 16, (bc + 4) * 16))
    v = vals.view(np.float16).astype(np.float64).reshape(-1, 16, 16)
    for r in range(br):
        for p in range(row_ptr[r], row_ptr[r + 1]):
            Ad[r * 16:(r + 1) * 16, col_idx[p] * 16:(col_idx[p] + 1) * 16] += v[p]
    Bd = np.zeros(((bc + 4) * 16, N))
    Bd[:K] = B
    want = (Ad @ Bd)[:M]
    absC = (np.abs(Ad) @ np.abs(Bd))[:M]
    hb, dA = _dev_bsr(S, torch, M, K, row_ptr, col_idx, vals)
    for rg, tiles in ((4, 4), (8, 8)):
        say(f"panel identity union order={order} row_group={rg} tiles={tiles}")
        C = S.spmm_wmma_opts(dA, torch.from_numpy(B16.view(np.int16)).cuda(),
                             S.BsrOptsT(rg, tiles, 0, 4)).cpu().numpy()
        check_csr(C, want, absC, tol=1e-5)


def test_panel_wide_matrix_identity(S, O, torch):
    # K beyond the union bitmap (8192 block-columns): identity union
    A = S.generate_uniform_random_csr(48, 140000, 0.0004, 12)
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(np.random.default_rng(13).uniform(-1, 1, (140000, 64)).astype(np.float32))
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    assert hb.block_cols > 8192
    for rg in (4, 8):
        say(f"panel wide K={A.num_cols} row_group={rg}")
        C = S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(),
                             S.BsrOptsT(rg, 4, 0, 2)).cpu().numpy()
        check_bsr(C, C32, absC)
        check_csr(C, C64, absC, tol=1e-5)


@pytest.mark.parametrize("rg,tiles,depth", [(4, 4, 2), (4, 4, 4), (4, 8, 2), (4, 8, 4),
                                            (8, 4, 4), (8, 8, 2), (8, 8, 4)])
@pytest.mark.parametrize("cfg", ["c3", "c4"])
def test_panel_configs(S, O, torch, rg, tiles, depth, cfg):
    A, B = make_config(S, cfg)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    say(f"panel config={cfg} row_group={rg} tiles={tiles} depth={depth}")
    C = S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(),
                         S.BsrOptsT(rg, tiles, 0, depth)).cpu().numpy()
    check_bsr(C, C32, absC)
    check_csr(C, C64, absC, tol=1e-5)


def test_panel_structured_shapes(S, O, torch):
    # banded and block-diagonal matrices whose blocks straddle block-rows,
    # ragged M / K, a partial last column tile (N = 200), and a union that
    # takes several 126-slot passes (dense block-rows, K = 6000)
    rng = np.random.default_rng(21)
    mats = [("banded_hb3", S.generate_banded_csr(200, 200, 3, 1), 200),
            ("banded_hb100", S.generate_banded_csr(1000, 1030, 100, 2), 128),
            ("block_diag_40", S.generate_block_diagonal_csr(500, 500, 40, 3, 1.0), 64),
            ("block_diag_256_n200", S.generate_block_diagonal_csr(1024, 1024, 256, 4, 1.0), 200),
            ("dense_rows_k6000", S.generate_uniform_random_csr(70, 6000, 0.2, 5), 64)]
    for name, A, N in mats:
        A.values = S.round_to_fp16(A.values)
        B = S.round_to_fp16(rng.uniform(-1, 1, (A.num_cols, N)).astype(np.float32))
        hb, B16, C32, C64, absC = _refs(S, O, A, B)
        for rg, tiles, depth in ((4, 4, 4), (4, 8, 2), (8, 8, 4), (0, 0, 0)):
            say(f"panel {name} N={N} row_group={rg} tiles={tiles} depth={depth}")
            C = S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(),
                                 S.BsrOptsT(rg, tiles, 0, depth)).cpu().numpy()
            check_bsr(C, C32, absC)
            check_csr(C, C64, absC, tol=1e-5)


def test_wmma_c_alignment(S, O, torch):
    # The record kernel writes C in 16-byte row chunks when C is 16-byte
    # aligned and in single floats otherwise: both give the same bits.
    A, B = _cases(S)["block_diag_small"]
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    dA = S.DeviceBSR(hb)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    M, N = hb.num_rows, B16.shape[1]
    for tiles in (1, 2, 4):
        aligned = torch.full((M, N), float("nan"), device="cuda")
        flat = torch.full((M * N + 1,), float("nan"), device="cuda")
        shifted = flat[1:].view(M, N)  # 4 bytes past a 16-byte boundary
        assert shifted.data_ptr() % 16 == 4
        say(f"wmma C alignment tiles={tiles}")
        S.spmm_wmma_opts(dA, dB, S.BsrOptsT(1, tiles, 0, 2), aligned)
        S.spmm_wmma_opts(dA, dB, S.BsrOptsT(1, tiles, 0, 2), shifted)
        torch.cuda.synchronize()
        a, b = aligned.cpu().numpy(), shifted.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.isnan(flat[0].item())  # nothing written before C
        check_bsr(a, C32, absC)


@pytest.mark.parametrize("N", [8, 24, 40, 72])
def test_wmma_partial_column_tiles(S, O, torch, N):
    # N % 8 == 0 but not a multiple of the 16 * tiles columns a wave covers:
    # the record kernel's 16-byte row-chunk C stores skip the chunks past N
    # (rows past M too: M = 45 leaves a partial last block-row)
    rng = np.random.default_rng(40 + N)
    A = S.generate_uniform_random_csr(45, 70, 0.1, 9)
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(rng.uniform(-1, 1, (70, N)).astype(np.float32))
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    dA = S.DeviceBSR(hb)
    dB = torch.from_numpy(B16.view(np.int16)).cuda()
    for tiles in (1, 2, 4):
        say(f"wmma partial tiles N={N} tiles={tiles}")
        C = torch.full((45, N), float("nan"), device="cuda")
        S.spmm_wmma_opts(dA, dB, S.BsrOptsT(1, tiles, 0, 2), C)
        torch.cuda.synchronize()
        got = C.cpu().numpy()
        check_bsr(got, C32, absC)
        check_csr(got, C64, absC, tol=1e-5)


def test_wmma_bad_row_group(S, torch):
    A = S.generate_banded_csr(64, 64, 3, 1)
    dA = S.DeviceBSR(S.bsr_from_csr_host(A))
    B16 = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(S.SpmmError) as e:
        S.spmm_wmma_opts(dA, B16, S.BsrOptsT(2, 0, 0, 0))
    assert e.value.code == S.SPMM_INVALID


@pytest.mark.parametrize("xcd_order", [1, 2])
def test_wmma_workgroup_orders(S, O, torch, xcd_order):
    # both workgroup -> tile maps of the wave kernel cover every tile once,
    # also when the workgroup count is not a multiple of the 8 XCDs
    cases = _cases(S)
    for name in ("ragged_dims", "n_not_16", "empty_block_rows", "wide_n", "block_diag_small"):
        A, B = cases[name]
        hb, B16, C32, C64, absC = _refs(S, O, A, B)
        for tiles in (1, 2, 4):
            say(f"wmma xcd_order={xcd_order} tiles={tiles} case={name}")
            C = S.spmm_wmma_opts(S.DeviceBSR(hb), torch.from_numpy(B16.view(np.int16)).cuda(),
                                 S.BsrOptsT(0, tiles, 1, 2, xcd_order)).cpu().numpy()
            check_bsr(C, C32, absC)
            check_csr(C, C64, absC, tol=1e-5)


@pytest.mark.parametrize("cfg", ["c3", "c4"])
def test_wmma_configs(S, O, torch, cfg):
    A, B = make_config(S, cfg)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    say(f"wmma config={cfg} blocks={hb.num_blocks} N={B.shape[1]}")
    C = _run_wmma(S, torch, hb, B16)
    rel = check_bsr(C, C32, absC)
    check_csr(C, C64, absC, tol=1e-5)
    say(f"  rel_l2 vs fp32 oracle={rel:.3e}")


def test_wmma_on_uniform_c1(S, O, torch):
    # high fill-in input (about 92 stored elements per nonzero) is still exact
    A, B = make_config(S, "c1")
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(B)
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    say(f"wmma config=c1 blocks={hb.num_blocks}")
    check_bsr(_run_wmma(S, torch, hb, B16), C32, absC)


def test_wmma_default_four_tiles_four_pairs(S, O, torch):
    # 1024 block-rows of ~127 blocks at N = 64: the default picks four column
    # tiles per wave and four pairs in flight
    A = S.generate_uniform_random_csr(16384, 2048, 0.02, 41)
    A.values = S.round_to_fp16(A.values)
    B = S.round_to_fp16(np.random.default_rng(42).uniform(-1, 1, (2048, 64)).astype(np.float32))
    hb, B16, C32, C64, absC = _refs(S, O, A, B)
    assert hb.num_blocks / hb.block_rows >= 96
    say(f"wmma default 4x4 blocks={hb.num_blocks}")
    C = _run_wmma(S, torch, hb, B16)
    check_bsr(C, C32, absC)
    check_csr(C, C64, absC, tol=1e-5)


def test_float_to_half_bitwise(S, O, torch):
    rng = np.random.default_rng(17)
    x = np.concatenate([rng.standard_normal(100003).astype(np.float32) * s
                        for s in (1e-6, 1e-3, 1.0, 1e3, 7e4)])
    x[:8] = [0.0, -0.0, 65504.0, 65520.0, 1e-8, 5.9604645e-08, 2.9802322e-08, -1.0009766]
    want = O.f32_to_f16(x)
    src = torch.from_numpy(x).cuda()
    say(f"float_to_half n={x.size} aligned")
    got = S.float_to_half(src).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, want)
    say("float_to_half unaligned view")
    sub = src[1:]  # 4-byte aligned only: scalar path
    got2 = S.float_to_half(sub).cpu().numpy().view(np.uint16)
    assert np.array_equal(got2, want[1:])


def test_wmma_argument_errors(S, torch):
    import ctypes
    s = S.BsrT(16, 16, 2, 1, 0, 0, 0, 0, 0)  # block_rows inconsistent with num_rows
    assert S.lib().spmm_c_wmma(ctypes.byref(s), 0, 0, 16, None) == S.SPMM_INVALID


def test_wmma_linearity_c4(S, O, torch):
    A, B = make_config(S, "c4")
    hb = S.bsr_from_csr_host(A)
    dA = S.DeviceBSR(hb)
    B16 = torch.from_numpy(O.f32_to_f16(B).view(np.int16)).cuda().view(torch.float16)
    say("wmma linearity c4")
    c1 = S.spmm_wmma(dA, B16)
    c2 = S.spmm_wmma(dA, B16 * 2)
    assert torch.equal(c2, c1 * 2)
