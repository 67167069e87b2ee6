"""bench_parallel (oracle path) and gpu_lock: CPU tests.

The sharding / aggregation cases restate the reference's
tests/test_oracle_sharding.py:95-420 against this module; the worker
protocol is driven with a fake worker script (no GPU, no torch in the
workers); the lock cases follow scripts/gpu_lock.py's behaviour.
"""
import json
import os
import sys
import textwrap
import threading
import time
from pathlib import Path

import pytest

import bench_parallel as bp
import gpu_lock
from conftest import CANONICAL, REPRO_IDS, VARIANT_IDS
from oracle_harness import _INVALID_STATUSES


# ---------------------------------------------------------------------------
# Task keys and expansion
# ---------------------------------------------------------------------------

def test_task_key_roundtrip():
    key = bp._make_shape_task_key("repros/canonical/r", "s0=8")
    assert key == "repros/canonical/r::SHAPE::s0=8"
    assert bp._split_shape_task_key(key) == ("repros/canonical/r", "s0=8")
    key = bp._make_shape_task_key("d", bp._DEFAULT_SHAPE_TOKEN)
    assert bp._split_shape_task_key(key) == ("d", "__default__")
    assert bp._split_shape_task_key("repros/canonical/r") == ("repros/canonical/r", None)
    # the label is everything after the LAST separator
    assert bp._split_shape_task_key("a::SHAPE::b::SHAPE::c") == ("a::SHAPE::b", "c")


def test_dir_and_display_names():
    key = bp._make_shape_task_key("repros/canonical/myrepro", "s0=8")
    assert bp._oracle_dir_name(key) == "myrepro"
    assert bp._oracle_dir_name("repros/canonical/myrepro") == "myrepro"
    assert bp._oracle_dir_name("repros/canonical/myrepro/repro.py") == "myrepro"
    assert bp._task_display_name(key) == "myrepro[s0=8]"
    assert bp._task_display_name(
        bp._make_shape_task_key("repros/canonical/myrepro", bp._DEFAULT_SHAPE_TOKEN)) == "myrepro"


def test_find_and_expand_the_canonical_dirs():
    dirs = bp.find_oracle_dirs([CANONICAL])
    assert sorted(d.name for d in dirs) == sorted(REPRO_IDS + VARIANT_IDS)
    tasks = bp._expand_oracle_shape_tasks(dirs)
    # three shapes.json points per BASELINE repro (BASELINE size + two
    # ragged); the corpus families carry the reference's points
    assert len(tasks) == (3 * len(REPRO_IDS) + 16 + 1 + 1 + 1 + 2 + 1 + 6 + 2 + 1 + 2
                          + 13 + 5 + 16 + 9 + 5 + 5
                          + 1 + 2 + 2 + 2 + 1 + 1 + 1 + 2 + 2 + 1 + 15)
    assert all("::SHAPE::" in t for t in tasks)
    from repro_harness import load_shape_configs
    for d in dirs:
        labels = list(load_shape_configs(str(d / "repro.py")))
        assert [bp._split_shape_task_key(t)[1] for t in tasks
                if bp._split_shape_task_key(t)[0] == str(d)] == labels


def test_withdrawn_points_are_no_oracle_for_shape():
    """A point its oracle.py withdraws (no registration matches it) is
    reported as NO_ORACLE_FOR_SHAPE before any check or timing runs; the
    dispatch miss needs no GPU."""
    from oracle_harness import _load_oracle_module
    from repro_harness import load_shape_configs
    seen = 0
    for rid in VARIANT_IDS:
        mod, _, d = _load_oracle_module(CANONICAL / rid)
        withdrawn = getattr(mod, "WITHDRAWN_POINTS", {})
        for label in load_shape_configs(str(d / "repro.py")):
            if label.rsplit("_", 1)[-1] in withdrawn:
                out = bp._bench_oracle_point(str(d), label, {"n_warmup": 1, "n_rep": 1,
                                                             "compile": False,
                                                             "skip_check": False})
                assert out[label]["status"] == "NO_ORACLE_FOR_SHAPE", out
                assert "NO_ORACLE_FOR_SHAPE" in _INVALID_STATUSES
                seen += 1
    assert seen == 18


def test_find_resolves_relative_dirs(monkeypatch):
    """Workers run from the package dir: a relative path on the command line
    must reach them as an absolute one."""
    monkeypatch.chdir(CANONICAL.parent)
    dirs = bp.find_oracle_dirs([Path("canonical") / REPRO_IDS[0]])
    assert [d.name for d in dirs] == [REPRO_IDS[0]] and dirs[0].is_absolute()


def test_expand_falls_back_to_default(monkeypatch, tmp_path):
    import repro_harness
    good, none, boom = tmp_path / "good", tmp_path / "none", tmp_path / "boom"

    def fake_load(repro_file, *a, **k):
        name = Path(repro_file).parent.name
        if name == "good":
            return {"s0=8": 1, "s0=16": 2}
        if name == "none":
            return {}
        raise RuntimeError("bad shapes.json")

    monkeypatch.setattr(repro_harness, "load_shape_configs", fake_load)
    assert bp._expand_oracle_shape_tasks([good, none, boom]) == [
        f"{good}::SHAPE::s0=8", f"{good}::SHAPE::s0=16",
        f"{none}::SHAPE::__default__", f"{boom}::SHAPE::__default__"]


def test_sort_big_dirs_first():
    tasks = ([bp._make_shape_task_key("small", "a")]
             + [bp._make_shape_task_key("big", s) for s in "abc"]
             + [bp._make_shape_task_key("mid", s) for s in "ab"])
    out = bp._sort_shape_tasks_big_dirs_first(tasks)
    assert [bp._split_shape_task_key(t)[0] for t in out] == ["big"] * 3 + ["mid"] * 2 + ["small"]
    assert [bp._split_shape_task_key(t)[1] for t in out[:3]] == ["a", "b", "c"]  # stable


# ---------------------------------------------------------------------------
# Aggregation (reference tests/test_oracle_sharding.py:195-420)
# ---------------------------------------------------------------------------

def _pt(status, us, cus):
    return {"status": status, "oracle_us": us, "compile_us": cus,
            "ratio": None if us is None or cus is None else cus / us}


def _per_dir():
    return {
        "/r/canonical/dirA/repro.py": {
            "modA_aaaa1111": _pt("GOOD", 10.0, 20.0),
            "modA_bbbb2222": _pt("GOOD", 30.0, 40.0),
            "modA_cccc3333": _pt("BAD_ORACLE", 99.0, 50.0),
        },
        "/r/canonical/dirB/repro.py": {"modB_dddd4444": _pt("UNVERIFIED_NUMERICS", 5.0, 6.0)},
    }


def _per_shape():
    k = bp._make_shape_task_key
    return {
        k("/r/canonical/dirA", "s0=8"): {"modA_aaaa1111": _pt("GOOD", 10.0, 20.0)},
        k("/r/canonical/dirA", "s0=16"): {"modA_bbbb2222": _pt("GOOD", 30.0, 40.0)},
        k("/r/canonical/dirA", "s0=32"): {"modA_cccc3333": _pt("BAD_ORACLE", 99.0, 50.0)},
        k("/r/canonical/dirB", "s0=8"): {"modB_dddd4444": _pt("UNVERIFIED_NUMERICS", 5.0, 6.0)},
    }


def test_aggregate_sharded_equals_unsharded():
    assert bp._aggregate_oracle_timings(_per_shape()) == bp._aggregate_oracle_timings(_per_dir())


def test_aggregate_contents():
    out = bp._aggregate_oracle_timings(_per_dir())
    a = out["dirA"]
    assert a["n_points"] == 2 and a["oracle_us"] == 20.0 and a["compile_us"] == 30.0
    assert a["points"]["modA_cccc3333"]["status"] == "BAD_ORACLE"
    assert set(a["points_by_shape"]) == {"aaaa1111", "bbbb2222", "cccc3333"}
    assert a["points_by_shape"]["aaaa1111"]["oracle_us"] == 10.0
    assert "dirB" not in out and out["__failures__"]["dirB"]["reason"] == "no_valid_point"


def test_aggregate_failure_reasons_and_oracle_only_is_a_floor():
    res = {
        "x/empty": {},
        "x/allbad": {"m_11111111": _pt("BAD_ORACLE", 5.0, 4.0)},
        "x/only": {"m_22222222": _pt("ORACLE_ONLY", 7.0, None)},
    }
    out = bp._aggregate_oracle_timings(res)
    assert out["__failures__"]["empty"]["reason"] == "no_points"
    assert out["__failures__"]["allbad"]["reason"] == "all_bad_oracle"
    # no compile comparator: a valid floor without compile_us
    assert out["only"]["oracle_us"] == 7.0 and "compile_us" not in out["only"]
    for status in _INVALID_STATUSES:
        o = bp._aggregate_oracle_timings({"x/d": {"m_3": _pt(status, 1.0, 2.0)}})
        assert o["__failures__"]["d"]["reason"] == "no_valid_point"


def test_points_by_shape_collision_prefers_valid_then_faster():
    res = {"x/d": {"modelA_abcd1234": _pt("UNVERIFIED_NUMERICS", 1.0, 2.0),
                   "modelB_abcd1234": _pt("GOOD", 9.0, 10.0),
                   "modelC_abcd1234": _pt("GOOD", 5.0, 10.0)}}
    out = bp._aggregate_oracle_timings(res)
    assert out["d"]["points_by_shape"]["abcd1234"]["oracle_us"] == 5.0
    assert out["d"]["oracle_us"] == 7.0  # median of the two valid points


def test_regroup_sharded_failures():
    k = bp._make_shape_task_key
    out = bp._regroup_sharded_oracle_failures({
        k("/r/canonical/dirA", "s0=8"): {"error": "boom-8"},
        k("/r/canonical/dirA", "s0=16"): {"error": "boom-16"},
        k("/r/canonical/dirB", "s0=4"): {"reason": "timeout"},
    })
    assert out["dirA"]["n_failed_shapes"] == 2
    assert sorted(out["dirA"]["failed_shapes"]) == ["s0=16", "s0=8"]
    assert out["dirA"]["example_error"] == "boom-8"
    assert out["dirB"]["example_error"] == "timeout"


def test_write_failure_matrix(tmp_path):
    k = bp._make_shape_task_key
    ok8 = {"modA_aaaa1111": _pt("GOOD", 10.0, 20.0)}
    ok16 = {"modA_bbbb2222": _pt("GOOD", 30.0, 40.0)}
    # (a) partial loss: still priced, shape_failures annotation, no __failures__
    t = bp._write_oracle_timings_output(
        tmp_path / "a" / "o.json", {k("/r/dirA", "s0=8"): ok8, k("/r/dirA", "s0=16"): ok16},
        {k("/r/dirA", "s0=32"): {"error": "OOM on s0=32"}})
    assert t["dirA"]["n_points"] == 2 and t["dirA"]["shape_failures"]["failed_shapes"] == ["s0=32"]
    assert "__failures__" not in t
    assert json.loads((tmp_path / "a" / "o.json").read_text()) == t
    # (b) invalid point + raised shapes: folded into the no_valid_point entry
    t = bp._write_oracle_timings_output(
        tmp_path / "b.json",
        {k("/r/dirB", "s0=8"): {"modB_dddd4444": _pt("UNVERIFIED_NUMERICS", 5.0, 6.0)}},
        {k("/r/dirB", "s0=16"): {"error": "r16"}, k("/r/dirB", "s0=32"): {"error": "r32"}})
    f = t["__failures__"]["dirB"]
    assert f["reason"] == "no_valid_point" and f["shape_failures"]["n_failed_shapes"] == 2
    # (c) every shape raised
    t = bp._write_oracle_timings_output(
        tmp_path / "c.json", {}, {k("/r/dirC", "s0=8"): {"error": "x"},
                                  k("/r/dirC", "s0=16"): {"error": "y"}})
    assert t["__failures__"]["dirC"]["reason"] == "all_shapes_failed"
    assert t["__failures__"]["dirC"]["n_failed_shapes"] == 2
    # (d) no failures: identical to the pure aggregate, byte-identical on disk
    res = {k("/r/dirA", "s0=8"): ok8, k("/r/dirA", "s0=16"): ok16}
    pure = bp._aggregate_oracle_timings(res)
    assert bp._write_oracle_timings_output(tmp_path / "d1.json", res, None) == pure
    assert bp._write_oracle_timings_output(tmp_path / "d2.json", res, {}) == pure
    assert (tmp_path / "d1.json").read_bytes() == (tmp_path / "d2.json").read_bytes()


# ---------------------------------------------------------------------------
# Worker count, GPU filter, clock pinning
# ---------------------------------------------------------------------------

def test_worker_count():
    assert bp._compute_worker_count(num_tasks=18, num_gpus=1, max_workers=None,
                                    workers_per_gpu=None) == (1, 1)
    assert bp._compute_worker_count(num_tasks=18, num_gpus=4, max_workers=None,
                                    workers_per_gpu=2) == (8, 2)
    assert bp._compute_worker_count(num_tasks=3, num_gpus=4, max_workers=None,
                                    workers_per_gpu=2) == (3, 2)
    assert bp._compute_worker_count(num_tasks=18, num_gpus=2, max_workers=3,
                                    workers_per_gpu=None) == (3, 2)
    assert bp._compute_worker_count(num_tasks=0, num_gpus=1, max_workers=None,
                                    workers_per_gpu=None) == (0, 1)
    with pytest.raises(ValueError):
        bp._compute_worker_count(num_tasks=1, num_gpus=0, max_workers=None, workers_per_gpu=None)
    with pytest.raises(ValueError):
        bp._compute_worker_count(num_tasks=1, num_gpus=1, max_workers=0, workers_per_gpu=None)


def test_filter_gpus():
    gpus = [{"index": str(i), "name": "AMD Instinct MI355X", "kind": "MI355X"} for i in range(4)]
    assert bp._filter_gpus(gpus, None) == gpus
    assert [g["index"] for g in bp._filter_gpus(gpus, "1, 3")] == ["1", "3"]
    assert bp._filter_gpus(gpus, " , ") == gpus


def test_clock_pinning_is_best_effort(monkeypatch, capsys):
    calls = []

    class R:
        def __init__(self, rc, err=""):
            self.returncode, self.stdout, self.stderr = rc, "", err

    def fake(cmd):
        calls.append(cmd)
        if cmd[-1] == "--resetperfdeterminism":
            return R(0)
        return R(0) if cmd[4] == "0" else (None if cmd[4] == "2" else R(1, "permission denied"))

    monkeypatch.setattr(bp, "_run_clock_cmd", fake)
    locked = bp._lock_gpu_clocks(["0", "1", "2"], 2100)
    assert locked == {"0"}
    assert calls[0] == ["sudo", "-n", "rocm-smi", "-d", "0", "--setperfdeterminism", "2100"]
    err = capsys.readouterr().err
    assert "permission denied" in err and "could not launch" in err
    bp._reset_gpu_clocks(locked)
    assert calls[-1] == ["sudo", "-n", "rocm-smi", "-d", "0", "--resetperfdeterminism"]


# ---------------------------------------------------------------------------
# Parent/worker protocol with a fake worker (no GPU)
# ---------------------------------------------------------------------------

FAKE_WORKER = textwrap.dedent(r'''
    import json, os, sys
    print("worker noise on stderr", file=sys.stderr, flush=True)
    for line in sys.stdin:
        t = line.strip()
        if not t or t == "EXIT":
            break
        if t.startswith("PREFETCH:"):
            continue
        label = t.rsplit("::SHAPE::", 1)[-1]
        if label.startswith("crash"):
            sys.exit(3)
        if label.startswith("deverr"):
            print("DEVICE_ERROR: HIP error: an illegal memory access was encountered", flush=True)
            sys.exit(1)
        if label.startswith("misalign"):
            print(json.dumps({"_repro": t + "-other", label: {}}), flush=True)
            continue
        if label.startswith("raise"):
            print(json.dumps({"_repro": t, "__error__": {"error": "ValueError: bad input",
                  "category": "runtime_error", "exception_type": "ValueError"}}), flush=True)
            continue
        print(json.dumps({"_repro": t, label: {"status": "ORACLE_ONLY", "oracle_us": 1.5,
                          "pid": os.getpid()}}), flush=True)
''')


def _fake_cmd(tmp_path):
    script = tmp_path / "fake_worker.py"
    script.write_text(FAKE_WORKER)
    return [sys.executable, "-u", str(script)]


def test_protocol_respawns_and_accounts_every_task(tmp_path):
    k = bp._make_shape_task_key
    tasks = [k("d/a", "p1"), k("d/a", "crash1"), k("d/a", "p2"), k("d/b", "deverr1"),
             k("d/b", "p3"), k("d/b", "misalign1"), k("d/c", "p4"), k("d/c", "raise1"),
             k("d/c", "p5")]
    gpus = [{"index": "0", "name": "fake", "kind": "FAKE"}]
    results, failures = bp.run_tasks(tasks, gpus, 1, _fake_cmd(tmp_path),
                                     env_for=lambda g: dict(os.environ))
    assert set(results) | set(failures) == set(tasks) and not set(results) & set(failures)
    assert set(results) == {k("d/a", "p1"), k("d/a", "p2"), k("d/b", "p3"),
                            k("d/c", "p4"), k("d/c", "p5")}
    assert "exited without a result" in failures[k("d/a", "crash1")]["error"]
    assert "worker noise" in failures[k("d/a", "crash1")]["error"]  # stderr tail kept
    assert failures[k("d/b", "deverr1")]["error"].startswith("DEVICE_ERROR")
    assert "misalignment" in failures[k("d/b", "misalign1")]["error"]
    assert failures[k("d/c", "raise1")]["exception_type"] == "ValueError"
    # a new process after the crash, the device error and the misalignment
    pids = [results[t][bp._split_shape_task_key(t)[1]]["pid"] for t in
            (k("d/a", "p1"), k("d/a", "p2"), k("d/b", "p3"), k("d/c", "p4"), k("d/c", "p5"))]
    assert len({pids[0], pids[1], pids[2], pids[3]}) == 4 and pids[3] == pids[4]


def test_protocol_two_workers_share_the_queue(tmp_path):
    k = bp._make_shape_task_key
    tasks = [k(f"d/x{i % 3}", f"p{i}") for i in range(12)]
    gpus = [{"index": "0", "name": "fake", "kind": "FAKE"},
            {"index": "1", "name": "fake", "kind": "FAKE"}]
    seen = []
    results, failures = bp.run_tasks(tasks, gpus, 2, _fake_cmd(tmp_path),
                                     env_for=lambda g: dict(os.environ),
                                     on_result=lambda r, n, t: seen.append((r["gpu"], n, t)))
    assert set(results) == set(tasks) and not failures
    assert {g for g, _, _ in seen} == {"0", "1"} and seen[-1][1:] == (12, 12)
    timed = bp._aggregate_oracle_timings(results)
    assert sorted(k for k in timed if not k.startswith("_")) == ["x0", "x1", "x2"]


def test_worker_env_pins_the_gpu(monkeypatch):
    monkeypatch.setenv("CUDA_VISIBLE_DEVICES", "5")
    env = bp._worker_env("3")
    assert env["HIP_VISIBLE_DEVICES"] == "3" and "CUDA_VISIBLE_DEVICES" not in env
    assert env["INDUCTOR_GPU_BENCH_LOCK"] == "1"
    assert str(bp.PKG_DIR) in env["PYTHONPATH"].split(os.pathsep)


def test_cli_requires_oracles():
    with pytest.raises(SystemExit):
        bp.main(["somewhere"])


# ---------------------------------------------------------------------------
# gpu_lock: discovery parsing and the lock protocol
# ---------------------------------------------------------------------------

def test_device_kinds_and_gfx_versions():
    assert gpu_lock.device_kind_from_name("AMD Instinct MI355X") == "MI355X"
    assert gpu_lock.device_kind_from_name("AMD Instinct MI300X OAM") == "MI300X"
    assert gpu_lock.device_kind_from_name("gfx950", "gfx950:sramecc+:xnack-") == "MI355X"
    assert gpu_lock.device_kind_from_name("Some GPU") == "Some_GPU"
    assert gpu_lock.gfx_from_target_version(90500) == "gfx950"
    assert gpu_lock.gfx_from_target_version(90402) == "gfx942"
    assert gpu_lock.gfx_from_target_version(90010) == "gfx90a"


def test_rocm_smi_json_parsing():
    text = json.dumps({
        "card1": {"Card Series": "AMD Instinct MI355X", "GFX Version": "gfx950", "Node ID": "3"},
        "card0": {"Card Series": "AMD Instinct MI355X", "GFX Version": "gfx950", "Node ID": "2"},
        "system": {"Driver version": "6.x"},
    })
    out = gpu_lock._parse_rocm_smi_json(text)
    assert [(d["index"], d["kind"], d["node"]) for d in out] == [("0", "MI355X", "2"),
                                                                  ("1", "MI355X", "3")]


def test_kfd_topology_discovery(tmp_path, monkeypatch):
    def node(i, simds, ver, name):
        d = tmp_path / str(i)
        d.mkdir()
        (d / "properties").write_text(f"cpu_cores_count 0\nsimd_count {simds}\n"
                                      f"gfx_target_version {ver}\n")
        (d / "name").write_text(name + "\n")
    node(0, 0, 0, "")              # CPU node
    node(2, 1024, 90500, "gfx950")
    node(1, 1024, 90500, "gfx950")
    out = gpu_lock._discover_kfd(tmp_path)
    assert [(d["index"], d["node"], d["kind"]) for d in out] == [("0", "1", "MI355X"),
                                                                  ("1", "2", "MI355X")]
    monkeypatch.setattr(gpu_lock, "_discover_kfd", lambda: out)
    monkeypatch.setattr(gpu_lock, "_discover_rocm_smi", lambda: [
        {"index": "0", "name": "AMD Instinct MI355X", "kind": "MI355X", "node": "2"}])
    env = {}
    got = gpu_lock.discover_gpus(env)
    assert got[1]["name"] == "AMD Instinct MI355X" and got[0]["name"] == "gfx950"
    assert [d["index"] for d in gpu_lock.discover_gpus({"HIP_VISIBLE_DEVICES": "1"})] == ["1"]
    rocr = gpu_lock.discover_gpus({"ROCR_VISIBLE_DEVICES": "1"})
    assert [(d["index"], d["node"]) for d in rocr] == [("0", "2")]
    monkeypatch.setattr(gpu_lock, "_discover_kfd", lambda: [])
    monkeypatch.setattr(gpu_lock, "_discover_rocm_smi", lambda: [])
    assert gpu_lock.discover_gpus({}) == [{"index": "0", "name": "UNKNOWN", "kind": "UNKNOWN"}]


def test_lock_metadata_and_exclusion(tmp_path):
    with gpu_lock.gpu_lock(3, lock_dir=tmp_path, label="bench x") as path:
        meta = gpu_lock.read_lock_metadata(path)
        assert meta["pid"] == str(os.getpid()) and meta["gpu"] == "3"
        assert meta["mode"] == "exclusive" and meta["label"] == "bench x"
        # a second exclusive holder (another open file description) times out
        with pytest.raises(TimeoutError, match="Timed out waiting for GPU 3 lock"):
            with gpu_lock.gpu_lock(3, lock_dir=tmp_path, timeout_s=0.2):
                pass
    with gpu_lock.gpu_shared_lock(3, lock_dir=tmp_path) as p1:
        with gpu_lock.gpu_shared_lock(3, lock_dir=tmp_path, timeout_s=0.5):
            assert gpu_lock.read_lock_metadata(p1)["mode"] == "shared"
        with pytest.raises(TimeoutError):
            with gpu_lock.gpu_lock(3, lock_dir=tmp_path, timeout_s=0.2):
                pass


def test_stale_holder_is_reported(tmp_path, monkeypatch):
    monkeypatch.setattr(gpu_lock, "STALE_LOCK_GRACE_S", 0.0)
    done = threading.Event()
    release = threading.Event()

    def holder():
        with gpu_lock.gpu_lock(0, lock_dir=tmp_path):
            # pretend the holder's process has died: a pid that cannot exist
            (tmp_path / "gpu_0.lock").write_text("pid=999999999\ngpu=0\nmode=exclusive\n")
            done.set()
            release.wait(5)

    th = threading.Thread(target=holder)
    th.start()
    done.wait(5)
    try:
        with pytest.raises(TimeoutError, match="stale"):
            with gpu_lock.gpu_lock(0, lock_dir=tmp_path, timeout_s=5):
                pass
    finally:
        release.set()
        th.join(5)


def test_lock_for_kind_picks_a_free_gpu(tmp_path):
    devs = [{"index": "0", "name": "AMD Instinct MI355X", "kind": "MI355X"},
            {"index": "1", "name": "AMD Instinct MI355X", "kind": "MI355X"}]
    with gpu_lock.gpu_lock(0, lock_dir=tmp_path):
        with gpu_lock.gpu_lock_for_kind("MI355X", lock_dir=tmp_path, devices=devs,
                                        timeout_s=2) as dev:
            assert dev["index"] == "1" and dev["lock_path"].endswith("gpu_1.lock")
    with pytest.raises(RuntimeError, match="No GPUs match"):
        with gpu_lock.gpu_lock_for_kind("MI300X", lock_dir=tmp_path, devices=devs):
            pass


def test_with_gpu_lock_cli_runs_the_command_pinned(tmp_path):
    out = tmp_path / "env.txt"
    rc = gpu_lock.main(["--gpu", "2", "--lock-dir", str(tmp_path), "--",
                        sys.executable, "-c",
                        f"import os; open({str(out)!r}, 'w').write(os.environ['HIP_VISIBLE_DEVICES'])"])
    assert rc == 0 and out.read_text() == "2"


# ---------------------------------------------------------------------------
# model_graph_accounting roll-up (reference tests/test_bench_accounting.py:1283-1418)
# ---------------------------------------------------------------------------

import model_graph_accounting as mga  # noqa: E402


def _occ(pattern_hash, shape_hash, n_ops=1):
    return mga.PartitionOccurrence(
        graph_name="full_graph_000.py", pattern_hash=pattern_hash, shape_hash=shape_hash,
        n_ops=n_ops, op_counts={"aten.add.Tensor": 1}, origin_ops=["aten.add.Tensor"],
        input_shapes=["[4]:f32"], max_output_shape=[4], has_reduction=False)


def _model(occs):
    ga = mga.GraphAccounting(graph_path="full_graph_000.py", graph_name="full_graph_000.py")
    ga.occurrences = list(occs)
    acc = mga.ModelAccounting(model_name="TinyModel", model_dir="/tmp/TinyModel")
    acc.graphs = [ga]
    return acc


def test_rollup_classifies_matched_fallback_and_unpriced():
    timing = {"oracle_us": 10.0, "compile_us": 9.0,
              "points_by_shape": {"shapeA": {"oracle_us": 5.0, "compile_us": 4.0}}}
    roll = mga._rollup_occurrence_timings(timing, [_occ("p", "shapeA"), _occ("p", "shapeB")])
    assert (roll["matched_occ"], roll["fallback_occ"], roll["unpriced_occ"], roll["total_occ"]) \
        == (1, 1, 0, 2)
    assert roll["mode"] == "partial" and roll["oracle_us_total"] == 15.0
    assert roll["compile_us_total"] == 13.0
    roll = mga._rollup_occurrence_timings(None, [_occ("p", "a"), _occ("p", "b")])
    assert roll["unpriced_occ"] == 2 and roll["mode"] == "untimed"
    assert roll["oracle_us_total"] is None
    # timed dir without a representative: a missing shape is unpriced, not 0
    roll = mga._rollup_occurrence_timings(
        {"points_by_shape": {"shapeA": {"oracle_us": 5.0}}}, [_occ("p", "shapeA"), _occ("p", "x")])
    assert (roll["matched_occ"], roll["fallback_occ"], roll["unpriced_occ"]) == (1, 0, 1)
    assert roll["oracle_us_total"] == 5.0
    # legacy timings (no points_by_shape): every occurrence at the dir number
    roll = mga._rollup_occurrence_timings({"oracle_us": 2.5}, [_occ("p", "a")] * 4)
    assert roll["mode"] == "legacy" and roll["oracle_us_total"] == 10.0
    assert roll["fallback_occ"] == 4


def test_model_report_gates_the_projection():
    timings = {"pointwise_priced": {"oracle_us": 7.0, "compile_us": 6.0,
                                    "points_by_shape": {"shapeA": {"oracle_us": 7.0,
                                                                   "compile_us": 6.0}}}}
    h2r = {"priced": "pointwise_priced", "untimed": "pointwise_untimed"}
    rep = mga.build_model_report(_model([_occ("priced", "shapeA"), _occ("priced", "shapeA"),
                                         _occ("untimed", "shapeC")]), h2r, timings, {})
    assert rep["projection_complete"] is False and rep["fusible_oracle_us_total"] is None
    assert rep["fusible_compile_us_total"] is None
    assert rep["fusible_oracle_us_total_is_lower_bound"] is True
    assert rep["fusible_oracle_us_total_partial"] == 14.0
    assert (rep["unpriced_occurrences"], rep["priced_occurrences"], rep["total_occurrences"]) \
        == (1, 2, 3)
    assert [k["pattern_hash"] for k in rep["unpriced_kernels"]] == ["untimed"]
    text = mga.format_text_report(rep)
    assert "INCOMPLETE" in text and "UNAVAILABLE" in text
    rep = mga.build_model_report(_model([_occ("priced", "shapeA")] * 2), h2r, timings, {})
    assert rep["projection_complete"] is True and rep["fusible_oracle_us_total"] == 14.0
    assert rep["fusible_oracle_us_total_is_lower_bound"] is False
    assert rep["unpriced_kernels"] == []


def test_occurrences_from_the_canonical_shapes(tmp_path):
    models = mga.collect_model_occurrences(CANONICAL)
    assert "baseline/config2_bias_gelu_nhwc" in models
    acc = models["baseline/config4a_residual_layernorm"]
    assert len(acc.all_occurrences) == 1
    occ = acc.all_occurrences[0]
    assert occ.pattern_hash == "var_mean_residual_layernorm" and occ.has_reduction
    h2r = mga.build_hash_to_repro(CANONICAL)
    assert h2r["var_mean_residual_layernorm"] == "var_mean_residual_layernorm"
    # a timings file shaped like bench_parallel's output prices it at its own shape
    timings = bp._aggregate_oracle_timings({
        bp._make_shape_task_key(str(CANONICAL / "var_mean_residual_layernorm"),
                                f"config4a_residual_layernorm_{occ.shape_hash}"):
            {f"config4a_residual_layernorm_{occ.shape_hash}":
                 {"status": "ORACLE_ONLY", "oracle_us": 89.4}}})
    path = tmp_path / "t.json"
    path.write_text(json.dumps(timings))
    rep = mga.build_model_report(acc, h2r, mga.load_timings(path))
    assert rep["projection_complete"] and rep["fusible_oracle_us_total"] == 89.4
    assert rep["matched_occurrences"] == 1
    # CLI over every model: the other five models have no timing -> INCOMPLETE
    out = tmp_path / "r.json"
    assert mga.main(["--all", "--json", "--timings", str(path), "--output", str(out)]) == 0
    reports = {r["model_name"]: r for r in json.loads(out.read_text())}
    assert reports["baseline/config4a_residual_layernorm"]["projection_complete"] is True
    assert reports["baseline/config1_row_mean"]["projection_complete"] is False
