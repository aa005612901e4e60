"""bench.py's host-side contract, on the CPU: the refusal of more than one GPU,
the measured-traffic figures it publishes only while they match the kernel
sources, and the algorithmic units of its roofline blocks
(scripts/roofline.py:177-185, harness.cu:239,278-280 of the reference)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "sparse-matrix-multiplication_amd"))

import bench  # noqa: E402
from spmm_amd import traffic  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_committed_traffic_matches_current_sources():
    # every pattern's capture is current: same source hash, same form
    forms = {"c1": ("csr", "rowgroups"), "c2": ("csr", "engine"), "c3": ("wmma", "tile"),
             "c4": ("wmma", "tile"), "c5": ("csr", "khalf")}
    for name, (backend, form) in forms.items():
        value, note = bench.load_traffic(name, backend, form)
        assert value is not None, f"{name}: {note}"
        assert value > 0 and "rocprofv3" in note


def test_stale_traffic_is_not_published(tmp_path, monkeypatch):
    # a capture taken on other sources, or on another launch form, is reported
    # as null with the reason
    src = os.path.join(ROOT, "profiles", "traffic_c2.json")
    with open(src) as f:
        t = json.load(f)
    prof = tmp_path / "profiles"
    prof.mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    t_stale = dict(t, sources_sha256="0" * 64)
    (prof / "traffic_c2.json").write_text(json.dumps(t_stale))
    value, note = bench.load_traffic("c2", "csr", "engine")
    assert value is None and note.startswith("stale")
    t = dict(t, sources_sha256=traffic.sources_sha256("csr"))  # current sources
    (prof / "traffic_c2.json").write_text(json.dumps(t))
    value, note = bench.load_traffic("c2", "csr", "split")
    assert value is None and "form" in note
    value, note = bench.load_traffic("c2", "csr", "engine")
    assert value == t["hbm_bytes_per_launch"]
    value, note = bench.load_traffic("c9", "csr", "engine")
    assert value is None and note == "no capture"


def test_source_hash_follows_the_kernel_text(tmp_path, monkeypatch):
    # the hash covers the kernel sources' names and code
    hip = tmp_path / "hip"
    hip.mkdir()
    for n in traffic.SOURCES["csr"]:
        (hip / n).write_text("a")
    monkeypatch.setattr(traffic, "HIP_DIR", str(hip))
    h1 = traffic.sources_sha256("csr")
    (hip / traffic.SOURCES["csr"][0]).write_text("b")
    assert traffic.sources_sha256("csr") != h1
    # comments and whitespace runs do not count; code does
    h2 = traffic.sources_sha256("csr")
    (hip / traffic.SOURCES["csr"][0]).write_text("b  // a note\n/* more */\n")
    assert traffic.sources_sha256("csr") == h2
    (hip / traffic.SOURCES["csr"][0]).write_text("b + 1")
    assert traffic.sources_sha256("csr") != h2


@pytest.mark.parametrize("backend", ["csr", "wmma"])
def test_roofline_units(backend):
    # c2 / c4 shapes: algorithmic bytes and the fractions follow the units
    if backend == "csr":
        P = {"name": "c2", "M": 8192, "K": 8192, "N": 128, "nnz": 671114, "desc": "",
             "backend": "csr", "form": "engine", "fill_in": 92.4, "dtype": "f32"}
        ms = 0.018
        blk, flops = bench.pattern_block(P, ms, None)
        alg = 8 * 671114 + 4 * 8193 + 4 * 8192 * 128 * 2
        assert blk["roofline"]["alg_bytes"] == alg == 13790292
        assert flops == 2 * 671114 * 128
        assert blk["roofline"]["frac"] == pytest.approx(alg / (ms * 1e-3) / 8e12, abs=1e-4)
    else:
        P = {"name": "c4", "M": 8192, "K": 8192, "N": 256, "nnz": 2097152, "desc": "",
             "backend": "wmma", "form": "wmma", "fill_in": 1.0, "dtype": "f16",
             "blocks": 8192}
        ms = 0.006
        blk, flops = bench.pattern_block(P, ms, 0.012)
        r = blk["roofline"]
        assert r["exec_flops"] == 2 * 256 * 8192 * 256
        assert r["hbm"]["alg_bytes"] == 516 * 8192 + 4 * 513 + 2 * 8192 * 256 + 4 * 8192 * 256
        assert r["frac"] == pytest.approx(r["exec_flops"] / (ms * 1e-3) / 2.5e15, abs=1e-4)
        assert blk["cold_ms_median"] == 0.012


def test_warm_up_counts():
    # an explicit --warmup is honoured exactly; the default warms for at least
    # 50 launches and WARM_S seconds and reports how many it ran
    class _Cuda:
        @staticmethod
        def synchronize():
            pass

    class _Torch:
        cuda = _Cuda()

    calls = []
    P = {"launch": lambda n: calls.append(n)}
    assert bench.warm_up(_Torch(), P, 7) == 7 and calls == [7]
    calls.clear()
    done = bench.warm_up(_Torch(), P, None, warm_s=0.02, chunk=10)
    assert done == sum(calls) and done >= 50 and calls[0] == 50
