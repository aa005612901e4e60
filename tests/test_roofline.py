"""MI355X roofline tool (spmm_amd.roofline): parsing, byte models and the
derived figures, against hand-computed values (CPU only)."""
import csv
import os

import pytest

import spmm_amd.roofline as R

LOG = """\
kernel=tiled_v3 m=8192 k=8192 n=128 nnz=671114 density=0.010000 time_ms=0.0174 gflops=9873.33 max_abs_err=1e-6
bsr_stats blocks=8192 stored_elems=2097152 original_nnz=2097152 fill_in_ratio=1.00 block_density=0.0312
kernel=wmma m=8192 k=8192 n=256 nnz=2097152 density=0.031250 time_ms=0.0073 gflops=148050.86
kernel=hybrid[wmma] m=8192 k=8192 n=256 nnz=2097152 density=0.031250 time_ms=0.0105 gflops=102475.84
hybrid_plan backend=wmma fill_in=1.00 reason="low BSR fill-in and N aligned to 16 -> Tensor Cores"
"""


def test_byte_models_match_the_formulas():
    # scripts/roofline.py:177-185 at c2: 8*nnz + 4*(M+1) + 4*K*N + 4*M*N
    assert R.csr_bytes(8192, 8192, 128, 671114) == 5368912 + 32772 + 4194304 + 4194304
    # BSR at c4: 516 per block + row pointers + fp16 B + fp32 C
    assert R.bsr_bytes(8192, 8192, 256, 8192) == 516 * 8192 + 4 * 513 + 2 * 8192 * 256 + \
        4 * 8192 * 256
    assert R.bsr_bytes(17, 5, 3, 1) == 516 + 4 * 3 + 2 * 15 + 4 * 51  # ceil-div block rows


def test_parse_attaches_block_counts_to_mfma_rows():
    rows = R.parse(LOG)
    assert [r["kernel"] for r in rows] == ["tiled_v3", "wmma", "hybrid[wmma]"]
    assert rows[0]["blocks"] is None
    assert rows[1]["blocks"] == 8192 and rows[2]["blocks"] == 8192
    assert rows[1]["time_ms"] == pytest.approx(0.0073) and rows[0]["nnz"] == 671114


def test_analyse_figures():
    res = {r["kernel"]: r for r in R.analyse(R.parse(LOG), gather_tbs=39.3)}
    c2 = res["tiled_v3"]
    flops = 2.0 * 671114 * 128
    b = 13790292.0
    assert c2["ai_flop_per_byte"] == pytest.approx(flops / b)
    assert c2["ceiling_gflops"] == pytest.approx(flops / b * 8000.0)  # HBM-bound: AI < ridge
    assert c2["eff_hbm_gbs"] == pytest.approx(b / (0.0174 * 1e6))
    assert c2["pct_hbm"] == pytest.approx(100 * b / (0.0174 * 1e6) / 8000.0)
    assert c2["bound"] == "hbm"
    # gather roof: 2 FLOPs per 4 gathered bytes per column -> 0.5 FLOP/B x 39.3 TB/s
    assert c2["gather_ceiling_gflops"] == pytest.approx(0.5 * 39300.0)
    c4 = res["wmma"]
    assert c4["exec_flops"] == 2.0 * 256 * 8192 * 256
    assert c4["pct_compute_peak"] == pytest.approx(
        100 * c4["exec_flops"] / 0.0073e-3 / 1e9 / R.MFMA_F16_GFLOPS)
    assert not c4["blocks_estimated"] and c4["bound"] == "hbm"


def test_mfma_row_without_stats_is_marked_estimated():
    rows = R.parse("kernel=wmma m=64 k=64 n=16 nnz=1000 time_ms=0.001 gflops=32.0\n")
    (r,) = R.analyse(rows)
    assert r["blocks_estimated"] and r["blocks"] == 4  # ceil(1000 / 256)


def test_cli_writes_csv_and_plot(tmp_path):
    log = tmp_path / "bench.log"
    log.write_text(LOG)
    out_csv = tmp_path / "roof.csv"
    out_png = tmp_path / "roof.png"
    assert R.main([str(log), "--csv", str(out_csv), "--plot", str(out_png)]) == 0
    with open(out_csv) as f:
        got = list(csv.DictReader(f))
    assert [g["kernel"] for g in got] == ["tiled_v3", "wmma", "hybrid[wmma]"]
    assert set(R.COLUMNS) <= set(got[0].keys())
    assert os.path.getsize(out_png) > 1000


def test_sweep_csv_input(tmp_path):
    p = tmp_path / "sweep.csv"
    p.write_text("pattern,kernel,m,k,n,nnz,density,time_ms,gflops\n"
                 "uniform,tiled_v3,4096,4096,128,167686,0.01,0.0079,5452.0\n")
    (r,) = R.analyse(R.parse_sweep_csv(str(p)))
    assert r["kernel"] == "tiled_v3" and r["hbm_bytes"] == R.csr_bytes(4096, 4096, 128, 167686)


def test_empty_input_fails(tmp_path):
    p = tmp_path / "empty.log"
    p.write_text("nothing here\n")
    assert R.main([str(p)]) == 1


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_roofline_rows.csv")


def test_byte_model_matches_the_reference_roofline_rows():
    # The reference's committed sweep (reports/data/sweep.csv, 108 rows over 9
    # kernels and 4 sizes) beside two columns its roofline script derived from
    # it (reports/data/roofline.csv, scripts/roofline.py:177-205): arithmetic
    # intensity and effective bandwidth depend only on the CSR byte model and
    # the measured time, not on the GPU.  A dropped row-pointer term, a 4-byte
    # instead of 8-byte entry or a fp16 B would each miss by far more than the
    # tolerance.
    rows = R.parse_sweep_csv(GOLDEN)
    with open(GOLDEN, newline="") as f:
        ref = list(csv.DictReader(f))
    assert len(rows) == len(ref) == 108
    res = R.analyse(rows)
    mfma = 0
    for row, r, g in zip(rows, res, ref):
        b = R.csr_bytes(row["m"], row["k"], row["n"], row["nnz"])
        ai, eff = float(g["ai_flop_per_byte"]), float(g["eff_dram_bw_gbs"])
        assert 2.0 * row["nnz"] * row["n"] / b == pytest.approx(ai, rel=1e-12)
        assert b / (row["time_ms"] * 1.0e6) == pytest.approx(eff, rel=1e-12)
        if R._is_mfma(row["kernel"]):
            mfma += 1  # priced on BSR bytes here, on CSR bytes in the reference
            continue
        assert r["ai_flop_per_byte"] == pytest.approx(ai, rel=1e-12)
        assert r["eff_hbm_gbs"] == pytest.approx(eff, rel=1e-12)
    assert mfma == 12
