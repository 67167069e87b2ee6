"""bench.py's one JSON line, as the round's driver reads it: the required
keys, one GPU, the roofline arithmetic (frac = achieved / peak, the
reference's memcopy SOL ratio), the CPU baseline's shape.  A short run of
the headline workload in a child process (the parent holds no bench state).
"""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

REQUIRED = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
            "roofline", "cpu_baseline")


@pytest.mark.gpu
def test_bench_json_line_contract():
    proc = subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), "--no-configs",
                           "--steps", "16", "--warmup", "4"],
                          cwd=ROOT, capture_output=True, text=True, timeout=220)
    assert proc.returncode == 0, proc.stderr[-3000:]
    lines = proc.stdout.strip().splitlines()
    assert len(lines) == 1, f"stdout must carry one JSON line, got {len(lines)}"
    line = json.loads(lines[0])
    missing = [k for k in REQUIRED if k not in line]
    assert not missing, missing
    assert line["n_gpus"] == 1 and line["steps"] == 16 and line["warmup"] == 4
    assert line["unit"] == "GB/s" and line["higher_is_better"] is True
    assert line["scaling"] == "weak" and line["vs_baseline"] is None
    assert line["config"]["workload"] and line["config"]["bytes_per_step"] == 411042304
    assert line["value"] > 0 and line["ms_per_step"] > 0
    rf = line["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["frac"] < 1 and abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    assert rf["traffic"] is None or rf["traffic"] >= line["config"]["bytes_per_step"]
    assert rf["memcopy_sol_us"] > 0
    assert abs(rf["vs_memcopy_sol"] - rf["memcopy_sol_us"] / rf["kernel_us"]) < 1e-3
    cb = line["cpu_baseline"]
    assert cb["kind"] in ("port", "reference") and cb["cores"] >= 1 and cb["value"] > 0
    assert cb["unit"] == "GB/s" and cb["sample"]


@pytest.mark.gpu
def test_pattern_copies_of_configs_4a_and_5():
    """The per-config pattern yardsticks: config 4a's two-in/two-out copy and
    config 5's hold copy time positive, the other configs have none."""
    sys.path.insert(0, str(ROOT))
    import bench
    from conftest import CANONICAL
    from repro_harness import load_shape_configs, make_inputs_from_config
    for rid in ("var_mean_residual_layernorm", "var_mean_batchnorm_train_relu", "mean_rmsnorm"):
        print(f"[pattern] {rid}", flush=True)
        cfg = next(iter(load_shape_configs(str(CANONICAL / rid / "repro.py")).values()))
        cpu_inputs = make_inputs_from_config(cfg, device="cpu")
        got = bench.pattern_copy_steady(rid, cpu_inputs, steps=8)
        if rid == "mean_rmsnorm":
            assert got is None
        else:
            name, us = got
            assert name and us > 0, got
