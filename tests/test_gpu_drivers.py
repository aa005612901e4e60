"""The command-line drivers on the GPU: spmm_bench (role of harness.cu), spmm_run
(role of spmm_run.cu) and the pattern sweep (role of run_pattern_sweep.py),
run as subprocesses and checked through the lines they print."""
import csv
import os
import re
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sparse-matrix-multiplication_amd")
BENCH = os.path.join(PKG, "build", "spmm_bench")
RUN = os.path.join(PKG, "build", "spmm_run")
KV = re.compile(r"(\w+)=(\S+)")
CSR_KERNELS = ("baseline", "memopt", "memopt_v2", "tiled", "tiled_v2", "tiled_v3", "tiled_v4")


def say(msg):
    print(msg, flush=True)


def _run(cmd, timeout=300):
    say("driver: " + " ".join(os.path.basename(c) if c.startswith("/") else c for c in cmd))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    return r


def _lines(stdout, prefix):
    return [dict(KV.findall(l)) for l in stdout.splitlines() if l.startswith(prefix)]


def test_bench_all_kernels_uniform():
    r = _run([BENCH, "--m", "512", "--k", "700", "--n", "128", "--density", "0.02",
              "--kernel", "all", "--warmup", "1", "--iters", "3", "--batch", "4",
              "--cpu-reps", "1"])
    assert r.returncode == 0, r.stderr
    recs = {d["kernel"]: d for d in _lines(r.stdout, "kernel=")}
    # 14 entries per row at N = 128: the hybrid's CSR side is the row groups
    assert set(recs) == set(CSR_KERNELS) | {"csr_auto[rowgroups]", "wmma", "hybrid[wmma]"} or \
        set(recs) == set(CSR_KERNELS) | {"csr_auto[rowgroups]", "wmma", "hybrid[csr]"}
    assert float(recs["csr_auto[rowgroups]"]["rel_l2_err"]) < 1e-6
    for k in CSR_KERNELS:
        d = recs[k]
        assert (d["m"], d["k"], d["n"]) == ("512", "700", "128")
        assert float(d["rel_l2_err"]) < 1e-6, (k, d["rel_l2_err"])
        assert float(d["time_ms"]) > 0 and float(d["cold_ms"]) > 0
        assert float(d["cpu_1t_ms"]) > 0 and int(d["cpu_threads"]) >= 1
    # fp16 rounding of fp32 inputs: the reference's wmma sits near 2.6e-4
    assert float(recs["wmma"]["rel_l2_err"]) < 1e-2
    assert "pct_mfma" in recs["wmma"]


@pytest.mark.parametrize("args,form", [
    (["--m", "2048", "--k", "2048", "--n", "256", "--density", "0.05"], "engine"),
    (["--m", "3000", "--k", "3000", "--n", "64", "--density", "0.01"], "rowgroups"),
    (["--m", "2048", "--k", "4096", "--n", "128", "--pattern", "power-law", "--mean-deg", "200",
      "--cap", "4096"], "split"),
    # B of 6 MiB: over one XCD's L2, half of it within
    (["--m", "2048", "--k", "12288", "--n", "128", "--pattern", "power-law", "--mean-deg", "200",
      "--cap", "4096"], "khalf"),
])
def test_bench_csr_auto(args, form):
    # the CSR form the hybrid picks, timed in batches: row groups, the engine
    # with the longest row as hint, or the merge-path partition for rows
    # longer than 2560 entries (over B-row halves when B is over 4 MiB and
    # half of it fits one XCD's L2)
    r = _run([BENCH] + args + ["--kernel", "csr_auto", "--warmup", "1", "--iters", "3",
                               "--batch", "4", "--cpu-reps", "1", "--no-cpu-1t"])
    assert r.returncode == 0, r.stderr
    d = _lines(r.stdout, "kernel=")[0]
    kinds = {"csr_auto[engine]", "csr_auto[rowgroups]", "csr_auto[split]", "csr_auto[khalf]"}
    assert d["kernel"] in kinds
    if form is not None:
        assert d["kernel"] == f"csr_auto[{form}]"
    assert float(d["rel_l2_err"]) < 1e-6 and float(d["cold_ms"]) > 0


@pytest.mark.parametrize("kernel", ["split", "khalf"])
def test_bench_forced_merge_path_forms(kernel):
    # the merge-path form and its B-row halves, whatever the hybrid would pick
    r = _run([BENCH, "--m", "2048", "--k", "12288", "--n", "128", "--pattern", "power-law",
              "--mean-deg", "200", "--cap", "4096", "--kernel", kernel, "--warmup", "1",
              "--iters", "3", "--batch", "4", "--cpu-reps", "1", "--no-cpu-1t"])
    assert r.returncode == 0, r.stderr
    d = _lines(r.stdout, "kernel=")[0]
    assert d["kernel"] == kernel and float(d["rel_l2_err"]) < 1e-6


def test_bench_khalf_refused_on_small_b():
    # B of 1 MiB fits one L2: the halves' plan refuses, the driver says so
    r = _run([BENCH, "--m", "512", "--k", "2048", "--n", "128", "--pattern", "power-law",
              "--mean-deg", "100", "--cap", "1500", "--kernel", "khalf", "--warmup", "1",
              "--iters", "2", "--batch", "2", "--cpu-reps", "1", "--no-cpu-1t"])
    assert r.returncode != 0 and "B-row halves plan failed" in r.stderr


def test_bench_wmma_exact_on_fp16_inputs():
    r = _run([BENCH, "--m", "512", "--k", "512", "--n", "64", "--pattern", "block-diagonal",
              "--block", "64", "--fp16-values", "--kernel", "wmma", "--warmup", "1",
              "--iters", "3", "--batch", "4", "--cpu-reps", "1"])
    assert r.returncode == 0, r.stderr
    stats = _lines(r.stdout, "bsr_stats")[0]
    assert stats["blocks"] == "128" and float(stats["fill_in_ratio"]) == 1.0
    d = _lines(r.stdout, "kernel=")[0]
    assert d["kernel"] == "wmma" and float(d["rel_l2_err"]) < 1e-6


def test_bench_tiled_v2_contract_skips():
    r = _run([BENCH, "--m", "256", "--k", "256", "--n", "96", "--kernel", "tiled_v2",
              "--iters", "1", "--batch", "1", "--cpu-reps", "1", "--no-cold", "--no-cpu-1t"])
    assert r.returncode == 0
    assert "tiled_v2 requires --n divisible by 128" in r.stderr
    assert not _lines(r.stdout, "kernel=")


@pytest.mark.parametrize("args,backend", [
    (["--m", "1024", "--k", "1024", "--n", "128"], "csr"),
    (["--m", "1024", "--k", "1024", "--n", "128", "--pattern", "banded",
      "--bandwidth", "40", "--fp16-values"], "wmma"),
    (["--m", "600", "--k", "900", "--n", "40", "--pattern", "banded"], "csr"),
])
def test_run_plan_and_pass(args, backend):
    r = _run([RUN, *args, "--warmup", "1", "--iters", "3"])
    assert r.returncode == 0, r.stderr
    plan = _lines(r.stdout, "plan ")[0]
    run = [l for l in r.stdout.splitlines() if l.startswith("run ")][0]
    assert plan["backend"] == backend
    assert f"mode=hybrid[{backend}]" in run
    assert "[PASS]" in run
    if "40" in args and args[args.index("40") - 1] == "--n":
        assert "N not a multiple of 16" in r.stdout


def test_run_reads_generated_bin(tmp_path):
    out = str(tmp_path / "pl.bin")
    env = dict(os.environ, PYTHONPATH=PKG)
    g = subprocess.run([sys.executable, "-m", "spmm_amd.gen_matrices", "--pattern", "power-law",
                        "--rows", "2000", "--cols", "1500", "--mean-deg", "24", "--out", out],
                       env=env, capture_output=True, text=True, timeout=300)
    assert g.returncode == 0, g.stderr
    nnz = re.search(r"nnz=(\d+)", g.stdout).group(1)
    r = _run([RUN, "--bin", out, "--n", "64", "--warmup", "1", "--iters", "2"])
    assert r.returncode == 0, r.stderr
    run = [l for l in r.stdout.splitlines() if l.startswith("run ")][0]
    d = dict(KV.findall(run))
    assert (d["m"], d["k"], d["nnz"]) == ("2000", "1500", nnz)
    assert "[PASS]" in run


def test_run_unified_mode():
    r = _run([RUN, "--m", "1024", "--k", "1024", "--n", "128", "--unified", "--warmup", "1",
              "--iters", "3"])
    assert r.returncode == 0, r.stderr
    run = [l for l in r.stdout.splitlines() if l.startswith("run ")][0]
    assert "mode=unified[csr]" in run and "[PASS]" in run


def test_bench_unified_kernel():
    r = _run([BENCH, "--m", "512", "--k", "512", "--n", "64", "--kernel", "unified",
              "--warmup", "1", "--iters", "3", "--cpu-reps", "1", "--no-cpu-1t"])
    assert r.returncode == 0, r.stderr
    d = _lines(r.stdout, "kernel=")[0]
    assert d["kernel"] == "unified" and float(d["rel_l2_err"]) < 1e-6


def test_run_rejects_multi_gpu():
    r = _run([RUN, "--multi-gpu"])
    assert r.returncode != 0 and "single-GPU" in r.stderr


def test_pattern_sweep_csv(tmp_path):
    env = dict(os.environ, PYTHONPATH=PKG)
    r = subprocess.run([sys.executable, "-m", "spmm_amd.run_pattern_sweep", "--sizes", "256",
                        "512", "--n", "128", "--warmup", "1", "--iters", "2", "--cwd",
                        str(tmp_path), "--extra", "--bench-args",
                        "--batch 2 --cpu-reps 1 --no-cold --no-cpu-1t"],
                       env=env, capture_output=True, text=True, timeout=600)
    say(r.stdout[-2000:])
    assert r.returncode == 0, r.stderr
    rows = list(csv.DictReader(open(tmp_path / "reports" / "data" / "pattern_sweep.csv")))
    assert list(rows[0])[:9] == ["pattern", "kernel", "m", "k", "n", "nnz", "density",
                                 "time_ms", "gflops"]
    patterns = {(row["pattern"], row["m"]) for row in rows}
    assert len(patterns) == 8
    for row in rows:
        if row["kernel"] in CSR_KERNELS:
            assert float(row["rel_l2_err"]) < 1e-6
        assert float(row["time_ms"]) > 0
