"""Headline benchmark: SpMM per BASELINE pattern at m = 8192 (c2 is `value`).

The metric is "SpMM GFLOP/s (2*nnz*N/t) + % HBM/MFMA roofline, m=8192 per
pattern".  `value` is c2 (uniform 8192 x 8192, density 0.01, N = 128, fp32),
the configuration the metric is quoted on; `patterns` holds one block per
BASELINE config (c1 .. c5), each timed the way spmm_hybrid_run runs it: the
backend hybrid_choose picks (reference spmm_hybrid.cu:32-56), and for CSR the
form the hybrid's CSR branch picks (row-block engine with the longest row as
hint, sub-wave row groups, the merge-path partition, or the merge-path
partition over B-row halves).

One step = one pass of the hot path over inputs already resident in HBM
(for the merge-path forms: the engine launch plus its fix-up; the B-row
halves' plan, built once from the host matrix, is outside the timed steps).  W untimed
steps (by default at least 50 and for at least 0.1 s, until the rate is
steady; `warmup` reports the count), then K steps back to back on torch's
current stream between two events on that stream, synchronised on both
sides.  With an explicit --warmup W the contract figure uses exactly W; the
steps then run well above their steady time (MI355X, --warmup 5 --steps 20:
c2 18.9 against 17.1 us, c1 8.0 against 5.9, c5 64.5 against 59.7; the
shader clock is already at 2.4 GHz, a copy kernel run first does not shorten
it, 2000 launches of the same step do), so
each block also carries `steady`: the same step after at least 0.1 s of
untimed launches, 500 timed, measured afterwards.  The gap is the shader
clock: `sclk_mhz` is the median shader clock the GPU delivers over the 200
launches right after the timed steps (and after the steady ones), sampled
every 5 us by a one-wave trace on a second stream (shader cycles against the
100 MHz real-time counter).  Under this load it starts near 2.1 GHz after
idle and reaches about 2.38 GHz only after ~1000 back-to-back launches while
the DPM state already reads 2.4 GHz (`--ramp c2,c1` prints time and clock per
batch of 20 launches from a fresh start).  `cold_ms_median` is the median of
single launches each preceded by a 512 MiB write that evicts L2 (4 MiB per
XCD) and the 256 MB MALL; warm is the contract figure.  `graph_ms_per_step`
is the same launches captured 100 at a time in one HIP graph and replayed (a
replay is first checked bit for bit against the eager result): what a caller
that captures its SpMM calls gets, reported beside the eager figure, never as
`value`.

Roofline units (scripts/roofline.py:177-185, harness.cu:239,278-280):
  CSR bytes = 8*nnz + 4*(M+1) + 4*K*N + 4*M*N, FLOPs = 2*nnz*N
  BSR bytes = 516*blocks + 4*(M/16+1) + 2*K*N + 4*M*N, executed MFMA FLOPs =
  2*256*blocks*N (GFLOP/s uses the original nnz, as the reference does).
`traffic` = HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE
(profiles/traffic_<cfg>.json, scaled by a plain-copy calibration), published
only while the kernel sources hash to what they were at capture; otherwise
null with the reason.  cpu_baseline times the CPU oracle (oracle/, test
infrastructure used here only as the reported baseline) on the same inputs on
all host threads this process may use (at most 16, the CPU share of one GPU on
the MI355X boxes) and on one thread.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "sparse-matrix-multiplication_amd")
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E datasheet
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA datasheet
COPY_BYTES = 256 * 1024 * 1024
FLUSH_BYTES = 512 * 1024 * 1024
WARM_S = 0.1  # seconds of untimed launches before timing, when --warmup is not given
STEADY_STEPS = 500  # timed steps of the steady-rate figure reported beside an explicit --warmup
METRIC = "SpMM GFLOP/s (2*nnz*N/t) + % HBM/MFMA roofline, m=8192 per pattern"
HEADLINE = "c2"
ORDER = ("c1", "c2", "c3", "c4", "c5")


def host_threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _median(v):
    v = sorted(v)
    return v[len(v) // 2]


def _time_cpu(fn, budget_s: float, min_runs: int):
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return _median(times), len(times)


def cpu_baseline(P, flops: float, budget_s: float = 2.5):
    """The oracle's loop on the same inputs: fp64-accumulated CSR x dense for
    CSR patterns, fp32 accumulation of the fp16 operands for BSR patterns."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np
    import oracle_lib as O
    if P["backend"] == "wmma":
        hb, B16 = P["host_bsr"], O.f32_to_f16(P["B"])
        kind = "oracle fp32-accumulate BSR x fp16 dense"

        def run(threads):
            return lambda: O.bsr_spmm_f32(P["M"], P["K"], hb.row_ptr, hb.col_idx, hb.values,
                                          B16, threads=threads)
    else:
        A = P["host"]
        rp = np.ascontiguousarray(A.row_ptr, np.int32)
        ci = np.ascontiguousarray(A.col_idx, np.int32)
        va = np.ascontiguousarray(A.values, np.float32)
        Bc = np.ascontiguousarray(P["B"], np.float32)
        kind = "oracle fp64-accumulate CSR x dense"

        def run(threads):
            return lambda: O.csr_spmm_f64(rp, ci, va, Bc, threads=threads, with_abs=False)
    T = host_threads()
    med_t, n_t = _time_cpu(run(T), budget_s, 3)
    med_1, n_1 = _time_cpu(run(1), budget_s, 1)
    return {"value": round(flops / med_t / 1e9, 2), "unit": "GFLOP/s", "cores": T,
            "kind": "port", "ms": round(med_t * 1e3, 3),
            "one_thread": {"value": round(flops / med_1 / 1e9, 2), "unit": "GFLOP/s",
                           "cores": 1, "ms": round(med_1 * 1e3, 3)},
            "sample": f"full {P['name']} workload ({kind}); median of {n_t} runs on {T} threads "
                      f"and of {n_1} on 1 thread; host reports {os.cpu_count()} CPUs, "
                      f"{len(os.sched_getaffinity(0))} in this process's affinity"}


def load_traffic(name: str, backend: str, kernel: str):
    """HBM bytes per launch for `name` if profiles/traffic_<name>.json was
    captured on the current kernel sources; else (None, reason)."""
    from spmm_amd.traffic import sources_sha256
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None, "no capture"
    with open(path) as f:
        t = json.load(f)
    if t.get("sources_sha256") != sources_sha256(backend):
        return None, f"stale: captured at {t.get('commit', '?')} on other kernel sources"
    if t.get("form") != kernel:
        return None, f"stale: captured on form {t.get('form')!r}, now {kernel!r}"
    return t.get("hbm_bytes_per_launch"), f"rocprofv3 FETCH_SIZE + WRITE_SIZE at {t.get('commit')}"


def build_pattern(S, torch, name: str):
    """Inputs in HBM and a launch(reps) closure for the form the hybrid picks."""
    from spmm_amd.configs import CONFIGS, make_config
    pattern, M, N, fp16, desc = CONFIGS[name]
    A, B = make_config(S, name)
    plan = S.hybrid_choose(A, N)
    cur = torch.cuda.current_stream  # launches go to the stream current at call time
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    P = {"name": name, "M": M, "K": A.num_cols, "N": N, "nnz": A.nnz, "host": A, "B": B,
         "desc": desc, "backend": plan.backend_name, "C": C,
         "fill_in": round(plan.fill_in_ratio, 4)}
    if plan.backend == S.BACKEND_WMMA:
        hb = S.bsr_from_csr_host(A)
        dA = S.DeviceBSR(hb)
        B16 = S.float_to_half(torch.from_numpy(B).cuda())
        P.update(host_bsr=hb, blocks=hb.num_blocks, dtype="f16 in, f32 accumulate")
        # spmm_hybrid_run's MFMA branch: the run-panel kernel when the block
        # structure is runs (its plan built with the BSR, outside the steps),
        # else the record kernel.
        try:
            tp = S.BsrTilePlan(dA)
        except S.SpmmError as e:
            if e.code != S.SPMM_UNSUPPORTED:
                raise
            tp = None
        if tp is not None:
            P["form"] = "tile"
            P["launch"] = lambda reps: tp.launch_repeat(B16, C, reps, stream=cur())
            P["keep"] = (dA, B16, tp)
        else:
            P["form"] = "wmma"
            P["launch"] = lambda reps: S.launch_repeat("wmma", dA, B16, C, reps, cur())
            P["keep"] = (dA, B16)
        return P
    form, opts, parts = S.csr_auto_form(A, N)
    dB = torch.from_numpy(B).cuda()
    P.update(form=form, dtype="f32")
    if form == "khalf":
        kp = S.KHalfPlan(A, N)
        P["launch"] = lambda reps: kp.launch_repeat(dB, C, reps, cur())
        P["keep"] = (kp, dB)
        return P
    dA = S.DeviceCSR(A)
    if form == "split":
        rows = torch.from_numpy(S.nnz_split_rows(A, parts)).cuda()
        carry = torch.empty((parts, N), dtype=torch.float32, device="cuda")
        P["parts"] = parts
        P["launch"] = lambda reps: S.launch_repeat_split(dA, rows, dB, C, carry, reps, cur())
        P["keep"] = (dA, dB, rows, carry)
    else:
        P["launch"] = lambda reps: S.launch_repeat_opts(dA, dB, C, opts, reps, cur())
        P["keep"] = (dA, dB)
    return P


def warm_up(torch, P, warmup, warm_s: float = WARM_S, chunk: int = 200) -> int:
    """Untimed launches before the timed ones: exactly `warmup` if given, else
    at least 50 and for at least `warm_s` seconds.  c2 needs about 2000
    launches to reach its steady rate (18.1 us per step after 50, 17.6 after
    500, 17.1 after 2000); c3 and c5 change by under 1%.  Returns the count."""
    if warmup is not None:
        P["launch"](max(warmup, 1))
        torch.cuda.synchronize()
        return max(warmup, 1)
    done = 50
    t0 = time.perf_counter()
    P["launch"](done)
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < warm_s:
        P["launch"](chunk)
        torch.cuda.synchronize()
        done += chunk
    return done


def time_warm(torch, P, steps: int) -> float:
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    P["launch"](steps)
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def clock_during(torch, S, P, launches: int, est_ms: float, interval_us: float = 5.0):
    """Median shader clock (MHz) the GPU delivers over `launches` back-to-back
    launches of the step: a one-wave trace on a second stream samples shader
    cycles against the 100 MHz real-time counter every `interval_us` while the
    launches run (S.shader_clock_trace).  Untimed."""
    side = torch.cuda.Stream()
    span_us = launches * est_ms * 1e3
    samples = int(span_us / interval_us) + 2
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        out = S.shader_clock_trace(samples, interval_us)
    P["launch"](launches)
    torch.cuda.synchronize()
    vals = [mhz for t, mhz in S.shader_clock_series(out) if t <= span_us]
    return round(_median(vals), 1) if vals else None


def ramp(torch, S, name: str, idle_s: float = 1.0, batches: int = 150, per: int = 20) -> dict:
    """Warm-up ramp of one pattern from this process's first launches: after
    one launch and `idle_s` seconds idle, `batches` batches of `per`
    back-to-back launches, each timed between two events while a one-wave
    shader-clock trace on a second stream samples the clock every 5 us (the
    batch's figure is the median over its intervals)."""
    P = build_pattern(S, torch, name)
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    P["launch"](1)
    e1.record(stream)
    torch.cuda.synchronize()
    est_us = e0.elapsed_time(e1) * 1e3
    time.sleep(idle_s)
    side = torch.cuda.Stream()
    us, mhz = [], []
    for _ in range(batches):
        span = est_us * per
        with torch.cuda.stream(side):
            out = S.shader_clock_trace(int(span / 5.0) + 2, 5.0)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        P["launch"](per)
        e1.record(stream)
        torch.cuda.synchronize()
        batch_us = e0.elapsed_time(e1) * 1e3
        vals = [m for t, m in S.shader_clock_series(out) if t <= batch_us]
        us.append(round(batch_us / per, 3))
        mhz.append(round(_median(vals), 1) if vals else None)
        est_us = batch_us / per
    return {"ramp": name, "form": P["form"], "idle_s": idle_s, "launches_per_batch": per,
            "us_per_launch": us, "sclk_mhz": mhz}


def time_cold(torch, P, flush, reps: int = 15) -> float:
    """Median of single launches, each after a 512 MiB write (L2 and MALL evicted)."""
    stream = torch.cuda.current_stream()
    evs = []
    for i in range(reps):
        flush.fill_(float(i))
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        P["launch"](1)
        e1.record(stream)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    return _median([a.elapsed_time(b) for a, b in evs])


def time_graph(torch, P, launches: int = 100, replays: int = 10):
    """Per-launch time when `launches` back-to-back launches are captured in
    one HIP graph and replayed (the device-side floor without the host's
    per-launch cost); also checks that a replay leaves the same C, bit for
    bit, as the eager launches.  Returns (ms, None) or (None, reason)."""
    C = P["C"]
    torch.cuda.synchronize()
    P["launch"](1)
    torch.cuda.synchronize()
    want = C.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        P["launch"](1)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g):
            P["launch"](launches)
    except Exception as e:  # capture refused: report, keep the eager figures
        torch.cuda.synchronize()
        return None, f"capture failed: {e}"[:200]
    C.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(C.view(torch.int32), want.view(torch.int32)):
        return None, "replay differs from the eager launches"
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    g.replay()
    e0.record(stream)
    for _ in range(replays):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (replays * launches)
    del g
    return ms, None


def pattern_block(P, ms: float, cold_ms: float):
    M, K, N, nnz = P["M"], P["K"], P["N"], P["nnz"]
    sec = ms * 1e-3
    flops = 2.0 * nnz * N
    blk = {"workload": P["desc"], "backend": P["backend"], "form": P["form"], "nnz": nnz,
           "N": N, "fill_in": P["fill_in"], "dtype": P["dtype"], "ms_per_step": round(ms, 6),
           "cold_ms_median": None if cold_ms is None else round(cold_ms, 6),
           "gflops": round(flops / sec / 1e9, 2)}
    if P["backend"] == "wmma":
        nb = P["blocks"]
        alg = 516.0 * nb + 4.0 * ((M + 15) // 16 + 1) + 2.0 * K * N + 4.0 * M * N
        exec_flops = 2.0 * 256 * nb * N
        tf = exec_flops / sec / 1e12
        hbm = alg / sec / 1e9
        traffic, note = load_traffic(P["name"], "wmma", P["form"])
        blk["blocks"] = nb
        blk["roofline"] = {"bound": "mfma", "achieved": round(tf, 2),
                           "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                           "exec_flops": exec_flops, "traffic": traffic, "traffic_source": note,
                           "hbm": {"achieved": round(hbm, 1), "peak": HBM_PEAK_GBS,
                                   "unit": "GB/s", "frac": round(hbm / HBM_PEAK_GBS, 4),
                                   "alg_bytes": alg}}
    else:
        alg = 8.0 * nnz + 4.0 * (M + 1) + 4.0 * K * N + 4.0 * M * N
        hbm = alg / sec / 1e9
        traffic, note = load_traffic(P["name"], "csr", P["form"])
        if "parts" in P:
            blk["parts"] = P["parts"]
        blk["roofline"] = {"bound": "hbm", "achieved": round(hbm, 1), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(hbm / HBM_PEAK_GBS, 4),
                           "alg_bytes": alg, "traffic": traffic, "traffic_source": note}
    return blk, flops


def measured_copy_gbs(torch, reps: int = 20) -> float:
    """HBM rate a plain 256 MiB device-to-device copy reaches on this GPU
    (read + write bytes per second), reported beside the datasheet peak."""
    stream = torch.cuda.current_stream()
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
    return 2.0 * COPY_BYTES / sec / 1e9


def copy_calibration(steps: int) -> int:
    """A plain copy of known size: reads and writes exactly COPY_BYTES per launch."""
    import torch
    torch.cuda.set_device(0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
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
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed launches per pattern (default: at least 50 and for at "
                         "least 0.1 s, until the rate is steady)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache timings")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the graph-replay timings (graph_ms_per_step)")
    ap.add_argument("--only", default="",
                    help="comma-separated subset of c1..c5 (profiling runs); the headline "
                         "line needs c2")
    ap.add_argument("--ramp", default="",
                    help="comma-separated patterns: print each one's warm-up ramp (time "
                         "per launch and delivered shader clock per batch of 20 launches "
                         "after 1 s idle) as one JSON line instead of the benchmark")
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
    names = [n for n in ORDER if not args.only or n in args.only.split(",")]

    sys.path.insert(0, PKG_DIR)
    import torch
    import spmm_amd as S

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    torch.cuda.set_device(0)
    S.lib()
    if args.ramp:
        for name in args.ramp.split(","):
            print(json.dumps(ramp(torch, S, name)), flush=True)
        return 0

    flush = None if args.no_cold else torch.empty(FLUSH_BYTES // 4, dtype=torch.float32,
                                                  device="cuda")
    blocks = {}
    for name in names:
        P = build_pattern(S, torch, name)
        warmed = warm_up(torch, P, args.warmup)
        ms = time_warm(torch, P, args.steps)
        sclk = {"next_200_launches": clock_during(torch, S, P, 200, ms)}
        cold = time_cold(torch, P, flush) if flush is not None else None
        blk, flops = pattern_block(P, ms, cold)
        blk["warmup_steps"] = warmed
        blk["sclk_mhz"] = sclk
        if not args.no_graph:
            gms, why = time_graph(torch, P)
            blk["graph_ms_per_step"] = None if gms is None else round(gms, 6)
            if why:
                blk["graph_note"] = why
        if args.warmup is not None:
            # The contract figure above used exactly --warmup untimed steps.  The
            # steady rate, after at least WARM_S of untimed launches, is measured
            # afterwards and reported beside it (never as ms_per_step or value).
            sw = warm_up(torch, P, None)
            sms = time_warm(torch, P, STEADY_STEPS)
            sclk["after_steady_next_200"] = clock_during(torch, S, P, 200, sms)
            blk["steady"] = {"ms_per_step": round(sms, 6),
                             "gflops": round(flops / (sms * 1e-3) / 1e9, 2),
                             "warmup_steps": sw, "steps": STEADY_STEPS}
        if not args.no_cpu:
            blk["cpu_baseline"] = cpu_baseline(P, flops)
        blocks[name] = blk
        print(f"bench: {name} {P['backend']}/{P['form']} {ms * 1e3:.2f} us warm "
              f"{(cold or 0) * 1e3:.2f} us cold {blk['gflops']:.0f} GFLOP/s", file=sys.stderr,
              flush=True)
        del P
    del flush
    if HEADLINE not in blocks:
        print(json.dumps({"patterns": blocks}), flush=True)
        return 0

    h = blocks[HEADLINE]
    copy_gbs = measured_copy_gbs(torch)
    roof = dict(h["roofline"])
    roof["measured_copy"] = {"value": round(copy_gbs, 1), "unit": "GB/s",
                             "frac": round(roof["achieved"] / copy_gbs, 4),
                             "what": "256 MiB device-to-device copy on this GPU, "
                                     "read + write bytes / time"}
    from spmm_amd.configs import CONFIGS
    _, M, N, _, desc = CONFIGS[HEADLINE]
    line = {
        "metric": METRIC,
        "value": h["gflops"],
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": h["warmup_steps"],
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (reference generator: mt19937 seed 42 Bernoulli CSR, seed 43 dense "
                "B; structured patterns from fixed seeds)",
        "config": {"workload": f"{HEADLINE}: {desc}, C = A*B fp32, the CSR form "
                               f"spmm_hybrid_run picks ({h['form']})",
                   "m": M, "k": M, "n": N, "density": 0.01, "seed_a": 42, "seed_b": 43,
                   "nnz": h["nnz"]},
        "roofline": roof,
        "cold_ms_median": h["cold_ms_median"],
    }
    if "steady" in h:
        line["steady"] = dict(h["steady"], what="the same step after at least "
                              f"{WARM_S} s of untimed launches, {STEADY_STEPS} timed, measured "
                              "after this line's own warmup + steps; not the contract figure")
    if "cpu_baseline" in h:
        line["cpu_baseline"] = h["cpu_baseline"]
    line["patterns"] = blocks
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
