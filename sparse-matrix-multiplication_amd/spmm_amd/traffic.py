"""HBM traffic per launch from rocprofv3 counter runs -> profiles/traffic_<cfg>.json.

Inputs are four `rocprofv3 --pmc <COUNTER> --output-format csv` output
directories: FETCH_SIZE and WRITE_SIZE over `bench.py --only <cfg> --no-cold
--no-cpu` (the engine's kernels), and the same two counters over
`bench.py --copy-calibration` (a plain copy that reads and writes exactly
268435456 bytes per launch).  Each engine counter (KiB per dispatch) is scaled
by known bytes / what the counter reads for the copy, then FETCH + WRITE gives
HBM bytes per launch.  The engine kernels of one step are the spmm:: kernels
dispatched once per step (the merge-path forms have two: the engine and its
fix-up), so set-up kernels dispatched once per run are left out.

The JSON records the hash of the kernel sources that decide what the launch
runs (`sources_sha256`, over their code with comments and whitespace runs
dropped); bench.py publishes the figure only while the current sources hash
the same.

    python -m spmm_amd.traffic --cfg c2 --form engine --fetch D1 --write D2 \
        --copy-fetch D3 --copy-write D4 --commit <git sha> --out profiles/traffic_c2.json
"""
from __future__ import annotations

import argparse
import csv
import glob
import hashlib
import re
import json
import os
from collections import defaultdict

HIP_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "csrc", "hip")
COPY_BYTES = 256 * 1024 * 1024

# Source files whose text decides what a pattern's launch runs, per backend.
SOURCES = {
    "csr": ("csr_kernels.hip", "hybrid.cpp", "khalf.cpp"),
    "wmma": ("bsr_kernels.hip", "bsr_tile.hip", "amdgcn.h"),
}


_COMMENT = re.compile(r"//[^\n]*|/\*.*?\*/", re.S)


def code_text(src: str) -> str:
    """The source without comments and with runs of whitespace collapsed: what
    the compiler sees, so a comment edit does not void a capture."""
    return " ".join(_COMMENT.sub(" ", src).split())


def sources_sha256(backend: str) -> str:
    h = hashlib.sha256()
    for name in SOURCES[backend]:
        p = os.path.join(HIP_DIR, name)
        if os.path.exists(p):
            h.update(name.encode())
            with open(p, encoding="utf-8") as f:
                h.update(code_text(f.read()).encode())
    return h.hexdigest()


def read_counter(directory: str, counter: str, name_filter: str):
    """{kernel name: [value per dispatch]} for one counter over every
    *counter_collection.csv under `directory` (values summed per dispatch)."""
    per = defaultdict(lambda: defaultdict(float))
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    for path in files:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                k = row.get("Kernel_Name", "")
                if name_filter and name_filter not in k:
                    continue
                per[k][(path, row.get("Dispatch_Id"))] += float(row["Counter_Value"])
    return {k: list(v.values()) for k, v in per.items()}


def per_step_kib(directory: str, counter: str):
    """Sum over the per-step spmm:: kernels of their mean KiB per dispatch."""
    got = read_counter(directory, counter, "spmm::")
    if not got:
        raise SystemExit(f"no spmm:: kernel with {counter} under {directory}")
    most = max(len(v) for v in got.values())
    step = {k: sum(v) / len(v) for k, v in got.items() if len(v) == most}
    return sum(step.values()), step, most


def copy_kib(directory: str, counter: str) -> float:
    got = read_counter(directory, counter, "")
    vals = [x for v in got.values() for x in v]
    if not vals:
        raise SystemExit(f"no {counter} values under {directory}")
    # the copy kernel is the dispatch with the largest count of bytes
    return max(vals)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--cfg", required=True)
    ap.add_argument("--form", required=True, help="launch form bench.py reports for the cfg")
    ap.add_argument("--backend", choices=sorted(SOURCES), default=None)
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--copy-fetch", required=True)
    ap.add_argument("--copy-write", required=True)
    ap.add_argument("--commit", required=True)
    ap.add_argument("--command", default="", help="the rocprofv3 command lines, for the record")
    ap.add_argument("--out", required=True)
    a = ap.parse_args()
    backend = a.backend or ("wmma" if a.form in ("wmma", "tile") else "csr")
    f_kib, f_step, n = per_step_kib(a.fetch, "FETCH_SIZE")
    w_kib, w_step, _ = per_step_kib(a.write, "WRITE_SIZE")
    cf, cw = copy_kib(a.copy_fetch, "FETCH_SIZE"), copy_kib(a.copy_write, "WRITE_SIZE")
    fs, ws = COPY_BYTES / (cf * 1024.0), COPY_BYTES / (cw * 1024.0)
    hbm = f_kib * 1024.0 * fs + w_kib * 1024.0 * ws
    out = {"cfg": a.cfg, "form": a.form, "commit": a.commit,
           "sources_sha256": sources_sha256(backend), "kernels": sorted(f_step),
           "dispatches_per_kernel": n,
           "fetch_size_kb_per_step": round(f_kib, 2), "write_size_kb_per_step": round(w_kib, 2),
           "copy_calibration": {"bytes": COPY_BYTES, "fetch_size_kb": cf, "write_size_kb": cw,
                                "fetch_scale": round(fs, 4), "write_scale": round(ws, 4)},
           "hbm_bytes_per_launch": int(round(hbm)), "commands": a.command}
    with open(a.out, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
