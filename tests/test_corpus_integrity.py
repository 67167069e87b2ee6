"""Static guards over the repository and its canonical dirs (no GPU).

* No in-process GPU timing outside the locked path (the reference's
  tests/test_no_unlocked_timing.py: an unlocked timing window is invalid,
  a co-tenant kernel inflates it).  Every real call of a timing primitive
  must sit in a file that takes the benchmark lock or delegates timing to
  the locked harness.
* Every shapes.json point of every canonical dir generates inputs with the
  point's exact shapes, strides and dtypes (the reference's
  tests/test_shapes_integrity.py: channels-last strides survive).
"""
import ast
import math
from pathlib import Path

import pytest
import torch

from conftest import CANONICAL, REPRO_IDS, VARIANT_IDS

ROOT = Path(__file__).resolve().parents[1]
SKIP_DIRS = {"tests", "_work", "gpurun_out", "__pycache__", ".git", "repros", "oracle"}
TIMING_NAMES = {"do_bench", "elapsed_time"}
# Substrings that put a file on the locked timing path: it takes the GPU lock
# itself or calls a harness entry point that does.
LOCK_MARKERS = ("_gpu_exclusive_lock", "gpu_lock", "INDUCTOR_GPU_BENCH_LOCK", "bench_oracle")


def _timing_calls(tree):
    hits = []
    for node in ast.walk(tree):
        if not isinstance(node, ast.Call):
            continue
        f = node.func
        name = f.id if isinstance(f, ast.Name) else f.attr if isinstance(f, ast.Attribute) else None
        if name in TIMING_NAMES:
            hits.append(f"{name}() line {node.lineno}")
    return hits


def _python_files():
    for p in ROOT.rglob("*.py"):
        if not any(part in SKIP_DIRS for part in p.relative_to(ROOT).parts):
            yield p


def test_no_unlocked_gpu_timing():
    offenders = []
    seen = 0
    for p in _python_files():
        src = p.read_text()
        hits = _timing_calls(ast.parse(src))
        if not hits:
            continue
        seen += 1
        if not any(m in src for m in LOCK_MARKERS):
            offenders.append(f"{p.relative_to(ROOT)}: {', '.join(hits)}")
    assert seen >= 2, "the scan found no timing call sites (bench.py, oracle_harness.py)"
    assert not offenders, "GPU timing outside the locked path:\n" + "\n".join(offenders)


def test_guard_flags_an_unlocked_timer():
    """Planted check: a file that times with events and takes no lock."""
    src = "import torch\ne0 = torch.cuda.Event(enable_timing=True)\nprint(e0.elapsed_time(e0))\n"
    assert _timing_calls(ast.parse(src)) and not any(m in src for m in LOCK_MARKERS)
    templated = "TEMPLATE = 'triton.testing.do_bench(fn)'\n"
    assert _timing_calls(ast.parse(templated)) == []  # string literals are not call sites


def _contiguous(shape):
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= max(d, 1)
    return tuple(reversed(st))


@pytest.mark.parametrize("rid", REPRO_IDS + VARIANT_IDS)
def test_generated_inputs_keep_point_layouts(rid):
    from input_codec import spec_from_compact
    from repro_harness import load_shape_configs, make_inputs_from_config
    import json
    points = json.loads((CANONICAL / rid / "shapes.json").read_text())["points"]
    cfgs = list(load_shape_configs(str(CANONICAL / rid / "repro.py")).values())
    assert len(cfgs) == len(points)
    for point, cfg in zip(points, cfgs):
        torch.manual_seed(1)
        made = make_inputs_from_config(cfg, device="meta")
        specs = [spec_from_compact(e) for e in point["inputs"]]
        assert len(made) == len(specs)
        for t, spec in zip(made, specs):
            if spec["kind"] != "tensor":
                assert list(t) == list(spec["dims"]), (rid, point["shape_hash"])
                continue
            assert tuple(t.shape) == tuple(spec["shape"]), (rid, point["shape_hash"])
            assert str(t.dtype) == f"torch.{spec['dtype']}", (rid, point["shape_hash"])
            want = tuple(spec["stride"]) if spec.get("stride") is not None else _contiguous(spec["shape"])
            assert t.stride() == want, (rid, point["shape_hash"], t.stride(), want)
            if t.dim() == 4 and want == tuple(
                    torch.empty(spec["shape"], device="meta",
                                memory_format=torch.channels_last).stride()) and math.prod(t.shape[1:2]) > 1:
                assert t.is_contiguous(memory_format=torch.channels_last)


# The reference's oracle-file contract (scripts/ORACLE_FORMAT.md:27, 64-72):
# the file opens with a one-sentence gap diagnosis whose classification is
# one of seven, naming what the oracle does, what Inductor does instead, why
# Inductor cannot do it today and the fix; and it does no sys.path surgery
# (the package comes from the environment -- PYTHONPATH here).
GAP_CLASSES = ("SCHEDULER_FUSION", "SCATTER_REDUCE", "COOPERATIVE_SPLIT_K",
               "ALGEBRAIC_ELIMINATION", "RECOMPUTE_FUSION", "BANDWIDTH_BOUND", "NEW_PATTERN")


@pytest.mark.parametrize("rid", REPRO_IDS + VARIANT_IDS)
def test_oracle_file_format(rid):
    import re
    src = (CANONICAL / rid / "oracle.py").read_text()
    first = src.splitlines()[0]
    m = re.match(r'"""Gap diagnosis \(classification: ([A-Z_]+)\): (.*)$', first)
    assert m, f"{rid}: oracle.py must open with the gap-diagnosis docstring, got {first[:80]!r}"
    cls, sentence = m.groups()
    assert cls in GAP_CLASSES, f"{rid}: classification {cls} is not one of {GAP_CLASSES}"
    assert sentence.startswith("this oracle ") and ", whereas Inductor " in sentence, rid
    assert "; Inductor cannot do this today because " in sentence, rid
    assert f"; the fix is {cls}: " in sentence, rid
    doc = ast.get_docstring(ast.parse(src))
    assert doc and doc.startswith("Gap diagnosis"), rid
    tree = ast.parse(src)
    for node in ast.walk(tree):
        if isinstance(node, ast.Attribute) and node.attr == "path" and \
                isinstance(node.value, ast.Name) and node.value.id == "sys":
            pytest.fail(f"{rid}: oracle.py touches sys.path (line {node.lineno})")
    assert "sys.path" not in src, f"{rid}: oracle.py mentions sys.path"
