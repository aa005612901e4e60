"""Performance sweep over sparsity patterns and sizes.

Counterpart of the reference's scripts/run_pattern_sweep.py (main :81-160):
for every (pattern, size) it writes a binary CSR with the generator CLI, runs
``spmm_bench --kernel all --bin FILE`` and collects every ``kernel=`` line into
one CSV with the reference's columns

    pattern,kernel,m,k,n,nnz,density,time_ms,gflops

so the reference's plotting scripts read it unchanged.  The per-pattern
generator parameters are the reference's fixed operating points
(run_pattern_sweep.py:48-53).  ``--extra`` appends this engine's additional
fields (cold_ms, pct_hbm, pct_mfma, rel_l2_err, cpu_ms, cpu_threads).

Usage (after ``make -C sparse-matrix-multiplication_amd``):
    python -m spmm_amd.run_pattern_sweep --sizes 1024 4096 --n 256
"""
from __future__ import annotations

import argparse
import csv
import os
import re
import subprocess
import sys

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEFAULT_BENCH = os.path.join(PKG_ROOT, "build", "spmm_bench")

# Generator flags per pattern, fixed across sizes so the pattern is the variable.
PATTERN_ARGS = {
    "uniform": ("--density", "0.01"),
    "banded": ("--bandwidth", "32"),
    "block-diagonal": ("--block", "16"),
    "power-law": ("--mean-deg", "32", "--alpha", "2.5"),
}

COLUMNS = ["pattern", "kernel", "m", "k", "n", "nnz", "density", "time_ms", "gflops"]
EXTRA_COLUMNS = ["cold_ms", "pct_hbm", "pct_mfma", "rel_l2_err", "cpu_ms", "cpu_threads"]

_KV = re.compile(r"(\w+)=(\S+)")
_INT_FIELDS = ("m", "k", "n", "nnz", "cpu_threads")
_STR_FIELDS = ("kernel",)


def parse_kernel_lines(text: str):
    """One dict per ``kernel=`` line of spmm_bench output (harness.cu:458-464)."""
    for line in text.splitlines():
        line = line.strip()
        if not line.startswith("kernel="):
            continue
        rec = {}
        try:
            for key, val in _KV.findall(line):
                if key in _STR_FIELDS:
                    rec[key] = val
                elif key in _INT_FIELDS:
                    rec[key] = int(val)
                else:
                    rec[key] = float(val)
        except ValueError:
            continue
        if not all(k in rec for k in ("kernel", "m", "k", "n", "nnz", "time_ms", "gflops")):
            continue  # a truncated line
        rec.setdefault("density", float("nan"))
        yield rec


def _gen_command(gen: str, pattern: str, m: int, seed: int, out: str):
    if gen.endswith(".py"):
        head = [sys.executable, gen]
    else:
        head = [sys.executable, "-m", gen]
    return head + ["--pattern", pattern, "--rows", str(m), "--cols", str(m), "--seed", str(seed),
                   *PATTERN_ARGS[pattern], "--out", out]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m spmm_amd.run_pattern_sweep", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--bench", default=DEFAULT_BENCH, help="spmm_bench binary")
    ap.add_argument("--gen", default="spmm_amd.gen_matrices",
                    help="generator: a module name or a .py script with the same CLI")
    ap.add_argument("--out", default="reports/data/pattern_sweep.csv")
    ap.add_argument("--datadir", default="data", help="where the .bin matrices are written")
    ap.add_argument("--patterns", nargs="+", default=list(PATTERN_ARGS))
    ap.add_argument("--sizes", nargs="+", type=int, default=[1024, 4096, 8192, 16384])
    ap.add_argument("--n", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--cwd", default=os.getcwd(), help="directory the paths are relative to")
    ap.add_argument("--extra", action="store_true", help="append this engine's extra fields")
    ap.add_argument("--bench-args", default="",
                    help="extra spmm_bench flags, e.g. '--no-cold --cpu-reps 1'")
    a = ap.parse_args(argv)

    cwd = os.path.abspath(a.cwd)
    bench = a.bench if os.path.isabs(a.bench) else os.path.join(cwd, a.bench)
    if not os.path.exists(bench):
        print(f"[error] benchmark binary {bench} not found; build it with "
              "`make -C sparse-matrix-multiplication_amd`", file=sys.stderr)
        return 1
    os.makedirs(os.path.join(cwd, a.datadir), exist_ok=True)
    env = dict(os.environ)
    env["PYTHONPATH"] = PKG_ROOT + os.pathsep + env.get("PYTHONPATH", "")

    rows = []
    for pattern in a.patterns:
        if pattern not in PATTERN_ARGS:
            print(f"[skip] unknown pattern {pattern!r}", file=sys.stderr)
            continue
        for m in a.sizes:
            binf = os.path.join(a.datadir, f"{pattern.replace('-', '')}_{m}.bin")
            g = subprocess.run(_gen_command(a.gen, pattern, m, a.seed, binf), cwd=cwd, env=env,
                               capture_output=True, text=True)
            print(g.stdout.strip() or f"generated {binf}", flush=True)
            if g.returncode != 0:
                print(f"[gen failed] {pattern} m={m}\n{g.stderr[-800:]}", file=sys.stderr)
                continue
            cmd = [bench, "--kernel", "all", "--bin", binf, "--n", str(a.n),
                   "--warmup", str(a.warmup), "--iters", str(a.iters), *a.bench_args.split()]
            b = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
            if b.returncode != 0:
                print(f"[bench failed] {pattern} m={m}\n{b.stderr[-800:]}", file=sys.stderr)
                continue
            got = 0
            for rec in parse_kernel_lines(b.stdout):
                rec["pattern"] = pattern
                rows.append(rec)
                got += 1
            print(f"  {pattern} m={m}: {got} kernel rows", flush=True)

    if not rows:
        print("[error] no rows collected; nothing written", file=sys.stderr)
        return 1
    out = os.path.join(cwd, a.out)
    os.makedirs(os.path.dirname(out) or ".", exist_ok=True)
    cols = COLUMNS + (EXTRA_COLUMNS if a.extra else [])
    with open(out, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols, extrasaction="ignore")
        w.writeheader()
        w.writerows(rows)
    print(f"\nWrote {a.out}  ({len(rows)} rows, {len(a.patterns)} patterns x "
          f"{len(a.sizes)} sizes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
