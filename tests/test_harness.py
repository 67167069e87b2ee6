"""oracle_harness host logic on the CPU: the fp64-anchored numerics gate,
the reviewed numerics opt-out, statuses and exit codes, the runner CLI, the
GPU lock, and static guards.  Restates the CPU-side cases of the
reference's tests/test_oracle_harness_hardening.py (gate :245-366, statuses
:376-381, opt-out loader/verdicts) and tests/test_bench_accounting.py:1420-1450
(lock metadata)."""
import ast
import json
import os
import re
import sys
import textwrap
from pathlib import Path

import pytest
import torch

import oracle_harness as oh
from oracle_harness import (_INVALID_STATUSES, _anchored_numerics_gate,
                            load_numerics_optout, numerics_optout_applies)

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "better-benchmark_amd"


# ---------------------------------------------------------------------------
# fp64-anchored gate
# ---------------------------------------------------------------------------

def t64(*v):
    return torch.tensor(v, dtype=torch.float64)


def t32(*v):
    return torch.tensor(v, dtype=torch.float32)


def test_gate_identical_outputs_pass():
    r = _anchored_numerics_gate([t32(1, 2, 3)], [t32(1, 2, 3)], [t64(1, 2, 3)], set())
    assert r["pass"] and r["per_output"][0]["err_oracle"] == 0.0


def test_gate_oracle_worse_than_compiled_fails():
    r = _anchored_numerics_gate([t32(1.1, 2.1, 3.1)], [t32(1, 2, 3)], [t64(1, 2, 3)], set())
    assert not r["pass"] and r["worst_output_idx"] == 0


def test_gate_small_errors_pass_and_absmax_scale():
    r = _anchored_numerics_gate([t32(1 + 2e-7, 2, 3)], [t32(1 + 1e-7, 2, 3)], [t64(1, 2, 3)], set())
    assert r["pass"]
    r = _anchored_numerics_gate([t32(1e6 + 5, 2e6 + 5)], [t32(1e6, 2e6)], [t64(1e6, 2e6)], set())
    assert r["pass"], "1e-5 * absmax term dominates"


def test_gate_skips_stochastic_and_non_float():
    r = _anchored_numerics_gate([t32(1), t32(0)], [t32(1), t32(99)], [t64(1), t64(99)], {1})
    assert r["pass"] and r["per_output"][1]["skip"] == "stochastic"
    i = torch.tensor([1, 2])
    r = _anchored_numerics_gate([i], [i], [i], set())
    assert r["per_output"][0]["skip"] == "non_float"


def test_gate_mixed_outputs_and_precision_record():
    r = _anchored_numerics_gate([t32(1, 2), t32(10.5, 20.5)], [t32(1, 2), t32(10, 20)],
                                [t64(1, 2), t64(10, 20)], set(), ref_precision="f32")
    assert not r["pass"] and r["per_output"][0]["pass"] and not r["per_output"][1]["pass"]
    assert r["ref_precision"] == "f32"


def test_gate_detects_exp2_substitution():
    x = torch.randn(1000, generator=torch.Generator().manual_seed(0)) * 3.0
    r = _anchored_numerics_gate([torch.exp2(x * 1.4426950408889634)], [torch.exp(x)],
                                [torch.exp(x.double())], set())
    e = r["per_output"][0]
    assert e["err_oracle"] > e["err_compiled"]


def test_invalid_statuses():
    # the reference's four, plus a kernel-recorded device fault (NaN outputs)
    assert _INVALID_STATUSES == {"UNVERIFIED_NUMERICS", "INVALID_CUDAGRAPH_WARNING",
                                 "NUMERICS_WORSE_THAN_COMPILED", "NO_ORACLE_FOR_SHAPE",
                                 "ORACLE_DEVICE_FAULT"}
    assert "ORACLE_ONLY" not in _INVALID_STATUSES
    assert "NUMERICS_OPTOUT_ACCEPTED" not in _INVALID_STATUSES


def test_cudagraph_warning_pattern():
    pat = oh._CUDAGRAPH_WARNING_PATTERNS
    for msg in ("CUDAGraph capture failed", "skipping cudagraphs due to", "hipGraph warning",
                "stream capture invalidated", "Graph capture ..."):
        assert pat.search(msg), msg
    assert not pat.search("tensor shapes differ")


# ---------------------------------------------------------------------------
# Numerics opt-out
# ---------------------------------------------------------------------------

def write_meta(tmp_path, opt):
    (tmp_path / "meta.json").write_text(json.dumps({"pattern_hash": "x", "numerics_optout": opt}))
    return tmp_path


def test_optout_loader(tmp_path):
    assert load_numerics_optout(tmp_path) is None
    d = write_meta(tmp_path, {"verified": True, "reason": "bf16 drift", "max_diff": 1e-3})
    assert load_numerics_optout(d)["reason"] == "bf16 drift"
    write_meta(tmp_path, {"verified": True, "reason": "  "})
    assert load_numerics_optout(tmp_path) is None
    write_meta(tmp_path, {"verified": False, "reason": "x"})
    assert load_numerics_optout(tmp_path) is None
    (tmp_path / "meta.json").write_text("{not json")
    assert load_numerics_optout(tmp_path) is None


def gate_result(err, absmax):
    return {"pass": False, "per_output": [{"idx": 0, "pass": False, "err_oracle": err,
                                           "ref_absmax": absmax}]}


def test_optout_verdicts():
    opt = {"verified": True, "reason": "bf16 rounding"}
    assert numerics_optout_applies(gate_result(3e-3, 1.0), opt)["accept"]
    assert not numerics_optout_applies(gate_result(0.5, 1.0), opt)["accept"]
    assert not numerics_optout_applies(gate_result(float("nan"), 1.0), opt)["accept"]
    assert not numerics_optout_applies(gate_result(float("inf"), 1.0), opt)["accept"]
    assert not numerics_optout_applies(gate_result(1e-3, 1.0), None)["accept"]
    assert not numerics_optout_applies(None, opt)["accept"]
    # bound floor: tiny reference scale still allows 1e-2 absolute
    assert numerics_optout_applies(gate_result(9e-3, 1e-6), opt)["accept"]


# ---------------------------------------------------------------------------
# Runner CLI on a fake canonical dir (CPU inputs)
# ---------------------------------------------------------------------------

REPRO = '''
import torch
from repro_harness import make_inputs_from_config, load_shape_configs
class Repro(torch.nn.Module):
    def forward(self, a, b):
        return (a * 2 + b, a.sum(-1))
def make_inputs(shape_config=None):
    cfg = shape_config or next(iter(load_shape_configs(__file__).values()))
    return make_inputs_from_config(cfg)
'''

ORACLE_OK = '''
import torch
from oracle_harness import oracle_impl
@oracle_impl(shapes="(T([6, 5], f32), T([6, 5], f32))")
def oracle_forward(inputs):
    a, b = inputs
    return (a * 2 + b, a.sum(-1))
'''

ORACLE_BAD = ORACLE_OK.replace("a * 2 + b", "a * 2 - b")
ORACLE_OTHER_SHAPE = ORACLE_OK.replace("[6, 5]", "[7, 5]")


def fake_dir(tmp_path, oracle_src):
    d = tmp_path / "repros" / "canonical" / "fake_pattern"
    d.mkdir(parents=True)
    (d / "repro.py").write_text(REPRO)
    (d / "oracle.py").write_text(textwrap.dedent(oracle_src))
    entry = [[6, 5], "f32", {"dev": "cpu"}]
    from repro_harness import shape_hash_of
    pts = [{"shape_hash": shape_hash_of([entry, entry]), "models": {"t/fake": {"occurrences": 1}},
            "inputs": [entry, entry]}]
    (d / "shapes.json").write_text(json.dumps({"points": pts}))
    return d


def test_runner_check_passes_and_fails(tmp_path, capsys):
    assert oh._runner_main([str(fake_dir(tmp_path / "ok", ORACLE_OK)), "--check"]) == 0
    assert oh._runner_main([str(fake_dir(tmp_path / "bad", ORACLE_BAD)), "--check"]) == 1
    out = capsys.readouterr().out
    assert "FAIL" in out and "PASS" in out


def test_runner_bench_gates_on_check(tmp_path, capsys):
    rc = oh._runner_main([str(fake_dir(tmp_path, ORACLE_BAD)), "--bench", "--no-compile",
                          "--disable-gpu-lock"])
    assert rc == 1
    assert "UNVERIFIED_NUMERICS" in capsys.readouterr().out


def test_runner_bench_cpu_path(tmp_path, capsys):
    rc = oh._runner_main([str(fake_dir(tmp_path, ORACLE_OK)), "--bench", "--rep", "3",
                          "--warmup", "1", "--disable-gpu-lock"])
    assert rc == 0
    out = capsys.readouterr().out
    summary = json.loads(out[out.rindex("\n{\n") + 1:])
    (bench,) = summary["bench"]
    assert bench["status"] in ("GOOD", "AT_FLOOR", "BAD_ORACLE") and bench["oracle_us"] > 0
    assert summary["check"] and all(summary["check"].values())


def test_runner_no_oracle_for_shape(tmp_path, capsys):
    rc = oh._runner_main([str(fake_dir(tmp_path, ORACLE_OTHER_SHAPE)), "--check"])
    assert rc == 1 and "NO_ORACLE_FOR_SHAPE" in capsys.readouterr().out


def test_check_oracle_catches_in_place_running_stats(tmp_path):
    """In-place outputs are compared on separate input sets (not skipped as
    stochastic): an oracle that forgets the running-stat update fails."""
    from conftest import CANONICAL
    import oracle as ref
    d = CANONICAL / "var_mean_batchnorm_train_relu"

    def good(inputs):
        x, g, b, rm, rv = inputs
        y, sm, si, rm2, rv2 = ref.batchnorm_train(x, g, b, rm, rv, momentum=0.1, eps=1e-5)
        rm.copy_(rm2)
        rv.copy_(rv2)
        return (y, sm, si, rm, rv)

    def forgets_update(inputs):
        x, g, b, rm, rv = inputs
        y, sm, si, _, _ = ref.batchnorm_train(x, g, b, rm, rv, momentum=0.1, eps=1e-5)
        return (y, sm, si, rm, rv)
    for fn in (good, forgets_update):
        fn.__module__ = "bn_test_module"
    kw = dict(point="222327da", device="cpu", atol=1e-5, rtol=1e-5)
    assert oh.check_oracle_all_shapes(good, d, "bn", **kw) == {"batchnorm_4x24x10x10_222327da": True}
    assert oh.check_oracle_all_shapes(forgets_update, d, "bn", **kw) == {
        "batchnorm_4x24x10x10_222327da": False}


# ---------------------------------------------------------------------------
# GPU lock
# ---------------------------------------------------------------------------

@pytest.fixture
def lock_env(tmp_path, monkeypatch):
    for v in ("INDUCTOR_GPU_BENCH_LOCK", "TORCHINDUCTOR_GPU_BENCH_LOCK", "HIP_VISIBLE_DEVICES",
              "ROCR_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES"):
        monkeypatch.delenv(v, raising=False)
    monkeypatch.setenv("INDUCTOR_GPU_BENCH_LOCK_DIR", str(tmp_path))
    return tmp_path


def test_lock_writes_metadata_and_nests(lock_env, monkeypatch):
    monkeypatch.setenv("HIP_VISIBLE_DEVICES", "3,1")
    with oh._gpu_exclusive_lock("label-x"):
        meta = (lock_env / "gpu_3.lock").read_text()
        assert f"pid={os.getpid()}" in meta and "gpu=3" in meta and "label=label-x" in meta
        with oh._gpu_exclusive_lock("nested"):
            assert "label=label-x" in (lock_env / "gpu_3.lock").read_text()
    assert (lock_env / "gpu_3.gate").exists()


def test_lock_disabled_and_forced(lock_env, monkeypatch):
    with oh._gpu_exclusive_lock("off", disabled=True):
        pass
    assert not (lock_env / "gpu_0.lock").exists()
    monkeypatch.setenv("INDUCTOR_GPU_BENCH_LOCK", "1")
    with oh._gpu_exclusive_lock("forced", disabled=True):
        assert "label=forced" in (lock_env / "gpu_0.lock").read_text()


def test_lock_device_precedence(lock_env, monkeypatch):
    monkeypatch.setenv("CUDA_VISIBLE_DEVICES", "5")
    assert oh._lock_gpu_id() == "5"
    monkeypatch.setenv("ROCR_VISIBLE_DEVICES", "2")
    assert oh._lock_gpu_id() == "2"
    monkeypatch.setenv("HIP_VISIBLE_DEVICES", "../7")
    assert oh._lock_gpu_id() == ".._7"


# ---------------------------------------------------------------------------
# Static guards
# ---------------------------------------------------------------------------

def product_python_files():
    return [p for p in PKG.rglob("*.py") if "_build" not in p.parts] + [ROOT / "bench.py"]


def test_timing_calls_sit_under_the_gpu_lock():
    """Every hipEvent elapsed_time call is in a file that takes the lock
    (reference: tests/test_no_unlocked_timing.py:107-139)."""
    for path in product_python_files():
        text = path.read_text()
        calls = [n for n in ast.walk(ast.parse(text))
                 if isinstance(n, ast.Call) and isinstance(n.func, ast.Attribute)
                 and n.func.attr == "elapsed_time"]
        if calls:
            assert "_gpu_exclusive_lock" in text, path


def test_product_never_imports_the_cpu_oracle():
    pat = re.compile(r"^\s*(import\s+oracle(\s|$|\.)|from\s+oracle(\s|\.))", re.M)
    for path in PKG.rglob("*.py"):
        assert not pat.search(path.read_text()), f"{path} imports the test oracle"
    for path in PKG.rglob("*.hip"):
        assert "hipo_ref" not in path.read_text()


MAIN_HOOK = '''
if __name__ == "__main__":
    from oracle_harness import oracle_main
    raise SystemExit(oracle_main(__file__, oracle_forward))
'''


def test_oracle_py_standalone_cli(tmp_path):
    """`python oracle.py [--check] [--bench] [--all-shapes]`: the reference
    template's CLI (scripts/oracle_template.py:147-237), run as __main__."""
    import os
    import subprocess
    pkg = Path(oh.__file__).resolve().parent
    env = dict(os.environ, PYTHONPATH=str(pkg))
    ok = fake_dir(tmp_path / "ok", ORACLE_OK + MAIN_HOOK)
    bad = fake_dir(tmp_path / "bad", ORACLE_BAD + MAIN_HOOK)

    def run(d, *args):
        return subprocess.run([sys.executable, str(d / "oracle.py"), *args],
                              capture_output=True, text=True, env=env, timeout=300)
    r = run(ok, "--check")
    assert r.returncode == 0 and "Correctness: PASS" in r.stdout, r.stderr[-2000:]
    r = run(bad, "--check", "--all-shapes")
    assert r.returncode == 1 and "Correctness: FAIL" in r.stdout
    r = run(ok, "--bench", "--rep", "3", "--warmup", "1", "--disable-gpu-lock", "--no-compile")
    assert r.returncode == 0, r.stderr[-2000:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["oracle_us"] > 0 and line["repro_id"] == "fake_pattern"
