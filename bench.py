"""Headline benchmark: CSR SpMM on BASELINE config c2 (uniform 8192 x 8192,
density 0.01, N = 128, fp32), the configuration the metric is quoted on.

One step = one pass of the hot path (one spmm_tiled_v3 launch, the CSR engine
the hybrid dispatcher picks for c2) over inputs already resident in HBM.
W untimed steps, then K steps launched back to back on torch's current stream
between two events on that stream (synchronised on both sides), through the
engine's C ABI.  Prints one JSON line.

roofline.achieved = compulsory bytes per launch (scripts/roofline.py:177-185:
8*nnz + 4*(M+1) + 4*K*N + 4*M*N) / average launch time.  roofline.traffic is the
HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
scaled by the copy-kernel calibration), read from profiles/traffic_c2.json when
present.  roofline.measured_copy is the rate a 256 MiB device-to-device copy
reaches on the same GPU, with achieved / that rate.  cpu_baseline times the CPU
oracle's fp64 loop (oracle/) on the same matrix on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "sparse-matrix-multiplication_amd")
HBM_PEAK_GBS = 8000.0
COPY_BYTES = 256 * 1024 * 1024

WORKLOAD = {"workload": "c2: uniform-random CSR 8192x8192 density 0.01, B 8192x128 fp32, "
                        "C = A*B fp32, kernel spmm_tiled_v3 (CSR engine)",
            "m": 8192, "k": 8192, "n": 128, "density": 0.01, "seed_a": 42, "seed_b": 43}


def cpu_baseline(A, B, flops: float, budget_s: float = 12.0):
    """Time the oracle's fp64 CSR loop (test infrastructure, used here only as
    the reported CPU baseline) on the same matrix, all host threads up to 16."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np
    import oracle_lib as O
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    rp = np.ascontiguousarray(A.row_ptr, np.int32)
    ci = np.ascontiguousarray(A.col_idx, np.int32)
    va = np.ascontiguousarray(A.values, np.float32)
    Bc = np.ascontiguousarray(B, np.float32)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        O.csr_spmm_f64(rp, ci, va, Bc, threads=threads, with_abs=False)
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": flops / med / 1e9, "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "sample": f"full c2 workload (oracle fp64 CSR x dense, {threads} threads), "
                      f"median of {len(times)} runs, {med * 1e3:.2f} ms each"}


def measured_copy_gbs(torch, stream, reps: int = 20) -> float:
    """HBM rate a plain 256 MiB device-to-device copy reaches on this GPU
    (read + write bytes per second): the measured counterpart of the 8 TB/s
    datasheet peak, reported beside it."""
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        dst.copy_(src)
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / reps
    del src, dst
    return 2.0 * COPY_BYTES / sec / 1e9


def copy_calibration(steps: int) -> int:
    """A plain copy of known size: reads and writes exactly COPY_BYTES per launch."""
    import torch
    torch.cuda.set_device(0)
    n = COPY_BYTES // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": COPY_BYTES, "launches": steps}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 256 MiB device-to-device copy, --steps times (the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.steps)
    if args.gpus != 1:
        print(f"bench.py: this SpMM engine runs on one GPU; --gpus {args.gpus} is not "
              "supported (the row-sharded multi-GPU split is a design note only)",
              file=sys.stderr)
        return 2

    sys.path.insert(0, PKG_DIR)
    import torch
    import spmm_amd as S

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    torch.cuda.set_device(0)
    S.lib()

    m, k, n = WORKLOAD["m"], WORKLOAD["k"], WORKLOAD["n"]
    A = S.generate_uniform_random_csr(m, k, WORKLOAD["density"], WORKLOAD["seed_a"])
    B = S.generate_dense_row_major(k, n, WORKLOAD["seed_b"])
    dA = S.DeviceCSR(A)
    dB = torch.from_numpy(B).cuda()
    dC = torch.empty((m, n), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()

    S.launch_repeat("tiled_v3", dA, dB, dC, max(args.warmup, 1), stream)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    S.launch_repeat("tiled_v3", dA, dB, dC, args.steps, stream)
    ev1.record(stream)
    torch.cuda.synchronize()
    total_ms = ev0.elapsed_time(ev1)
    ms = total_ms / args.steps

    nnz = A.nnz
    flops = 2.0 * nnz * n
    gflops = flops / (ms * 1e-3) / 1e9
    alg_bytes = 8.0 * nnz + 4.0 * (m + 1) + 4.0 * k * n + 4.0 * m * n
    achieved = alg_bytes / (ms * 1e-3) / 1e9

    copy_gbs = measured_copy_gbs(torch, stream)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_c2.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    line = {
        "metric": "SpMM GFLOP/s (2*nnz*N/t) + % HBM/MFMA roofline, m=8192 per pattern",
        "value": round(gflops, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (reference generator: mt19937 seed 42 Bernoulli CSR, seed 43 dense B)",
        "config": dict(WORKLOAD, nnz=nnz),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "measured_copy": {"value": round(copy_gbs, 1), "unit": "GB/s",
                                       "frac": round(achieved / copy_gbs, 4),
                                       "what": "256 MiB device-to-device copy on this GPU, "
                                               "read + write bytes / time"}},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(A, B, flops)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
