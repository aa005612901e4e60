"""bench.py end to end on the GPU, in this process: the JSON line's contract
keys, and that its figures follow from one another (value from c2's step time,
the roofline from the algorithmic bytes, the steady-rate figure beside an
explicit --warmup, the measured traffic present for both back ends)."""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

pytestmark = pytest.mark.gpu


def _close(a, b, rel=1e-3):
    return abs(a - b) <= rel * max(abs(a), abs(b))


def test_bench_line_is_consistent(S, monkeypatch, capsys):
    import bench
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "1", "--only", "c2,c3,c4", "--steps",
                                      "20", "--warmup", "5", "--no-cpu", "--no-cold",
                                      "--no-graph"])
    assert bench.main() == 0
    line = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "patterns", "steady"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 20 and line["warmup"] == 5
    assert line["unit"] == "GFLOP/s" and line["higher_is_better"] is True

    c2 = line["patterns"]["c2"]
    assert c2["form"] == "engine" and c2["N"] == 128
    assert line["value"] == c2["gflops"] and line["ms_per_step"] == c2["ms_per_step"]
    assert _close(c2["gflops"], 2.0 * c2["nnz"] * 128 / (c2["ms_per_step"] * 1e-3) / 1e9)

    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["peak"] == 8000.0
    assert _close(roof["achieved"], roof["alg_bytes"] / (line["ms_per_step"] * 1e-3) / 1e9)
    assert _close(roof["frac"], roof["achieved"] / roof["peak"], rel=2e-3)
    assert roof["traffic"] is not None and roof["traffic"] > roof["alg_bytes"]

    steady = line["steady"]
    assert steady["steps"] == 500 and steady["warmup_steps"] >= 50
    assert _close(steady["gflops"], 2.0 * c2["nnz"] * 128 / (steady["ms_per_step"] * 1e-3) / 1e9)

    c3 = line["patterns"]["c3"]
    assert c3["backend"] == "wmma" and c3["roofline"]["bound"] == "mfma"
    assert c3["roofline"]["traffic"] is not None
    assert _close(c3["roofline"]["achieved"],
                  c3["roofline"]["exec_flops"] / (c3["ms_per_step"] * 1e-3) / 1e12)
    assert "steady" in c3
    c4 = line["patterns"]["c4"]
    assert c3["form"] == "tile" and c4["form"] == "tile"  # the hybrid's run-panel form
    assert c4["roofline"]["traffic"] is not None
    for blk in line["patterns"].values():  # the delivered clock beside each timing
        clk = blk["sclk_mhz"]
        assert 100.0 < clk["next_200_launches"] < 3000.0
        assert 100.0 < clk["after_steady_next_200"] < 3000.0
