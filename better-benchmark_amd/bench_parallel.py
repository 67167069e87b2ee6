"""Parallel oracle benchmark runner for ROCm: `--oracles` mode of the
reference's scripts/bench_parallel.py.

    python -m bench_parallel repros/canonical --oracles [--gpus 0,1]
        [--output oracle_timings.json] [--n-warmup 25] [--n-rep 100]
        [--compile | --no-compile] [--oracle-skip-check] [--lock-clocks]

What it does (reference bench_parallel.py:2053-2680, oracle path):
  1. find every canonical dir with an oracle (oracle*.py beside repro.py)
     and expand it into one task per shapes.json point, keyed
     `<dir>::SHAPE::<label>` (`__default__` for a dir without points);
     dirs with the most points go first (no straggler tail);
  2. start persistent worker subprocesses, round-robin over the selected
     GPUs; each worker is pinned with HIP_VISIBLE_DEVICES and serialises its
     timing windows on the per-GPU lock (INDUCTOR_GPU_BENCH_LOCK=1);
  3. each task runs the point's numerics check
     (check_oracle_all_shapes(point=label)) then bench_oracle; a worker that
     hits a device error reports DEVICE_ERROR and exits, and the parent
     respawns it for the next task; results carry the task key back so a
     misaligned pipe is detected and the worker reset;
  4. results are aggregated per dir into the schema
     model_graph_accounting --timings reads: `points_by_shape` keyed by the
     shape hash, a median `oracle_us` / `compile_us` over valid points, and
     `__failures__` for dirs with no valid point or raised shapes.

ROCm specifics: GPU discovery and the pinning variable come from gpu_lock
(KFD topology + rocm-smi, HIP_VISIBLE_DEVICES); optional clock pinning uses
`rocm-smi --setperfdeterminism <MHz>` / `--resetperfdeterminism` (the
counterpart of `nvidia-smi -lgc` / `-rgc`), best effort and never fatal, off
by default (it needs root); device errors are recognised by HIP's messages.
The torch.compile (Inductor) comparator runs by default, as in the
reference's bench_oracle; `--no-compile` skips it (ORACLE_ONLY status, still
a valid floor).

Only the oracle path is provided: the reference's compile-path sweep,
full-graph mode, perf.json updates and merges are outside this backend.
"""
from __future__ import annotations

import argparse
import collections
import json
import os
import queue
import subprocess
import sys
import tempfile
import threading
import time
from collections import Counter
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent

_RESERVED_TOP_LEVEL_KEYS = {"_metadata", "__failures__", "__summary__"}
_RESERVED_RESULT_LABELS = {"__graph__"}
_SHAPE_TASK_SEP = "::SHAPE::"
_DEFAULT_SHAPE_TOKEN = "__default__"
#: Words in an exception message that mean the device context is unusable.
_DEVICE_ERROR_MARKERS = ("HIP error", "hipError", "CUDA error", "CUDA", "device-side assert",
                         "illegal memory access", "memory access fault",
                         "HSA_STATUS_ERROR")
#: Default clock for --lock-clocks on MI355X (a sustained engine-clock bin).
DEFAULT_LOCK_MHZ = 2100


# ---------------------------------------------------------------------------
# Task keys (reference :92-122, 145-224, 380-409)
# ---------------------------------------------------------------------------

def _normalize_shape_label(label: str) -> str:
    return "default" if label == _DEFAULT_SHAPE_TOKEN else label


def _make_shape_task_key(dir_path: str, shape_label: str) -> str:
    return f"{dir_path}{_SHAPE_TASK_SEP}{shape_label}"


def _split_shape_task_key(task_key: str) -> tuple[str, str | None]:
    """(dir, label) of a sharded key; (key, None) for a bare dir path."""
    if _SHAPE_TASK_SEP in task_key:
        dir_path, label = task_key.rsplit(_SHAPE_TASK_SEP, 1)
        return dir_path, label
    return task_key, None


def _oracle_dir_name(task_key: str) -> str:
    dir_part, _ = _split_shape_task_key(str(task_key))
    path = Path(dir_part)
    return path.parent.name if path.name == "repro.py" else path.name


def _task_display_name(task_key: str) -> str:
    dir_part, label = _split_shape_task_key(str(task_key))
    name = _oracle_dir_name(dir_part)
    if label is None or label == _DEFAULT_SHAPE_TOKEN:
        return name
    return f"{name}[{label}]"


def find_oracle_dirs(paths: list[Path]) -> list[Path]:
    """Canonical dirs holding an oracle (oracle*.py) next to a repro.py, as
    absolute paths (the workers run from the package dir)."""
    def has_oracle(d: Path) -> bool:
        return (d / "repro.py").is_file() and any(d.glob("oracle*.py"))

    out: list[Path] = []
    seen: set[str] = set()
    for p in paths:
        p = Path(p).resolve()
        cands = [p] if p.is_dir() and has_oracle(p) else (
            sorted({f.parent for f in p.rglob("repro.py")}) if p.is_dir() else
            [p.parent] if p.name == "repro.py" else [])
        for d in cands:
            if has_oracle(d) and str(d) not in seen:
                seen.add(str(d))
                out.append(d)
    return out


def _expand_oracle_shape_tasks(dirs: list[Path]) -> list[str]:
    """One task per shapes.json point; a dir without points (or whose
    points do not load) is one `__default__` task."""
    from repro_harness import load_shape_configs

    tasks: list[str] = []
    for d in dirs:
        try:
            configs = load_shape_configs(str(Path(d) / "repro.py"))
        except Exception:
            configs = None
        if configs:
            tasks.extend(_make_shape_task_key(str(d), label) for label in configs)
        else:
            tasks.append(_make_shape_task_key(str(d), _DEFAULT_SHAPE_TOKEN))
    return tasks


def _sort_shape_tasks_big_dirs_first(tasks: list[str]) -> list[str]:
    count = Counter(_split_shape_task_key(t)[0] for t in tasks)
    return sorted(tasks, key=lambda k: (-count[_split_shape_task_key(k)[0]],
                                        _split_shape_task_key(k)[0]))


# ---------------------------------------------------------------------------
# Aggregation into the model-accounting timings schema (reference :1242-1454)
# ---------------------------------------------------------------------------

def _median(values: list[float]) -> float:
    s = sorted(values)
    mid = len(s) // 2
    return s[mid] if len(s) % 2 else (s[mid - 1] + s[mid]) / 2.0


def _metric_result_items(results: dict):
    for label, result in results.items():
        if label not in _RESERVED_RESULT_LABELS and isinstance(result, dict):
            yield label, result


def _prefer_shape_point(candidate: dict, existing: dict, floor_excluded) -> bool:
    """A valid point beats an invalid one; of two valid points, the faster."""
    def valid(p):
        return (p.get("status") not in floor_excluded
                and isinstance(p.get("oracle_us"), (int, float)))
    cv, ev = valid(candidate), valid(existing)
    if cv != ev:
        return cv
    if cv:
        return candidate["oracle_us"] < existing["oracle_us"]
    return (isinstance(candidate.get("oracle_us"), (int, float))
            and not isinstance(existing.get("oracle_us"), (int, float)))


def _aggregate_oracle_timings(all_results: dict) -> dict:
    """{task key -> {label -> point}} -> {dir name -> priced entry}.

    Per dir: `points` (label -> oracle_us, compile_us, ratio, status),
    `points_by_shape` (trailing shape-hash token of the label -> the same
    plus the dispatch fallback flag; a collision keeps the better point),
    `oracle_us` / `compile_us` = medians over valid points (statuses outside
    _INVALID_STATUSES and not BAD_ORACLE), `n_points`.  A dir with no valid
    point goes to `__failures__` with reason no_points / all_bad_oracle /
    no_valid_point.  Sharded and per-dir payloads aggregate identically.
    """
    from oracle_harness import _INVALID_STATUSES

    floor_excluded = _INVALID_STATUSES | {"BAD_ORACLE"}
    merged: dict[str, dict] = {}
    for task_key, results in all_results.items():
        bucket = merged.setdefault(_oracle_dir_name(str(task_key)), {})
        if isinstance(results, dict):
            for label, point in results.items():
                if isinstance(point, dict):
                    bucket[label] = point

    flat: dict[str, dict] = {}
    failures: dict[str, dict] = {}
    for dir_name, results in merged.items():
        points: dict[str, dict] = {}
        by_shape: dict[str, dict] = {}
        valid_us: list[float] = []
        valid_compile: list[float] = []
        n_total = n_bad = 0
        for label, point in _metric_result_items(results):
            n_total += 1
            status = point.get("status")
            us = point.get("oracle_us")
            compile_us = point.get("compile_us")
            dispatch = point.get("dispatch")
            fallback = dispatch.get("fallback") if isinstance(dispatch, dict) else None
            points[label] = {"oracle_us": us, "compile_us": compile_us,
                             "ratio": point.get("ratio"), "status": status}
            entry = {**points[label], "fallback": fallback}
            shape_hash = label.rsplit("_", 1)[-1]
            if shape_hash not in by_shape or _prefer_shape_point(entry, by_shape[shape_hash],
                                                                 floor_excluded):
                by_shape[shape_hash] = entry
            if status == "BAD_ORACLE":
                n_bad += 1
            if status not in floor_excluded and isinstance(us, (int, float)):
                valid_us.append(us)
                if isinstance(compile_us, (int, float)):
                    valid_compile.append(compile_us)
        if not valid_us:
            reason = ("no_points" if n_total == 0 else
                      "all_bad_oracle" if n_bad == n_total else "no_valid_point")
            failures[dir_name] = {"reason": reason, "n_points": n_total,
                                  "n_bad_oracle": n_bad, "points": points}
            continue
        entry = {"oracle_us": round(_median(valid_us), 2), "n_points": len(valid_us),
                 "points": points, "points_by_shape": by_shape}
        if valid_compile:
            entry["compile_us"] = round(_median(valid_compile), 2)
        flat[dir_name] = entry
    if failures:
        flat["__failures__"] = failures
    return flat


def _regroup_sharded_oracle_failures(sharded_failures: dict) -> dict:
    """Worker exceptions keyed by task -> {dir name -> failed shapes}."""
    by_dir: dict[str, dict] = {}
    for task_key, failure in sharded_failures.items():
        dir_path, label = _split_shape_task_key(str(task_key))
        entry = by_dir.setdefault(_oracle_dir_name(dir_path),
                                  {"failed_shapes": [], "n_failed_shapes": 0,
                                   "example_error": None})
        if label is not None:
            entry["failed_shapes"].append(label)
        entry["n_failed_shapes"] += 1
        if entry["example_error"] is None and isinstance(failure, dict):
            entry["example_error"] = failure.get("error") or failure.get("reason")
    return by_dir


def _atomic_write_json(path: Path, payload: dict) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.NamedTemporaryFile("w", dir=path.parent, prefix=f".{path.name}.",
                                     suffix=".tmp", delete=False) as tmp:
        json.dump(payload, tmp, indent=2)
        tmp.write("\n")
        tmp_path = Path(tmp.name)
    os.replace(tmp_path, path)


def _write_oracle_timings_output(output_path: Path, all_results: dict,
                                 failures: dict | None = None) -> dict:
    """Aggregate and write; raised shapes annotate a still-priced dir
    (`shape_failures`) or fold into its `__failures__` entry, never vanish."""
    timed = _aggregate_oracle_timings(all_results)
    if failures:
        priced = {k for k in timed if k not in _RESERVED_TOP_LEVEL_KEYS}
        agg = timed.setdefault("__failures__", {})
        for dir_name, entry in _regroup_sharded_oracle_failures(failures).items():
            note = {"n_failed_shapes": entry["n_failed_shapes"],
                    "failed_shapes": entry["failed_shapes"],
                    "example_error": entry["example_error"]}
            if dir_name in priced:
                timed[dir_name]["shape_failures"] = note
            elif dir_name in agg:
                agg[dir_name].setdefault("shape_failures", note)
            else:
                agg[dir_name] = {"reason": "all_shapes_failed", **note}
        if not agg:
            timed.pop("__failures__", None)
    _atomic_write_json(output_path, timed)
    return timed


# ---------------------------------------------------------------------------
# GPUs, clocks, worker count (reference :680-870)
# ---------------------------------------------------------------------------

def _filter_gpus(gpus: list[dict], selected: str | None) -> list[dict]:
    if not selected:
        return gpus
    wanted = {s.strip() for s in selected.split(",") if s.strip()}
    return [g for g in gpus if g["index"] in wanted] if wanted else gpus


def _run_clock_cmd(cmd: list[str]):
    """Run a clock command without raising; None if it could not start."""
    try:
        return subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                              text=True, timeout=30)
    except Exception as exc:
        print(f"[clock-lock] WARNING: could not run {' '.join(cmd)}: "
              f"{type(exc).__name__}: {exc}", file=sys.stderr)
        return None


def _lock_gpu_clocks(indices: list[str], mhz: int) -> set[str]:
    """Best effort: cap each GPU's engine clock at `mhz` (performance
    determinism mode).  Returns the indices that accepted; only warns."""
    locked: set[str] = set()
    for idx in indices:
        res = _run_clock_cmd(["sudo", "-n", "rocm-smi", "-d", str(idx),
                              "--setperfdeterminism", str(mhz)])
        if res is not None and res.returncode == 0:
            locked.add(str(idx))
        else:
            detail = ((res.stderr or res.stdout or "").strip() if res is not None
                      else "could not launch sudo/rocm-smi")
            print(f"[clock-lock] WARNING: GPU {idx} not pinned to {mhz} MHz: "
                  f"{detail or 'non-zero exit'}", file=sys.stderr)
    print(f"[clock-lock] pinned {len(locked)}/{len(indices)} GPUs to {mhz} MHz"
          if locked else "[clock-lock] unavailable; running with default clocks",
          file=sys.stderr)
    return locked


def _reset_gpu_clocks(indices: set[str]) -> None:
    ok = 0
    for idx in sorted(indices):
        res = _run_clock_cmd(["sudo", "-n", "rocm-smi", "-d", str(idx),
                              "--resetperfdeterminism"])
        if res is not None and res.returncode == 0:
            ok += 1
        else:
            print(f"[clock-lock] WARNING: GPU {idx} clock reset failed", file=sys.stderr)
    if indices:
        print(f"[clock-lock] reset {ok}/{len(indices)} GPUs", file=sys.stderr)


def _compute_worker_count(*, num_tasks: int, num_gpus: int, max_workers: int | None,
                          workers_per_gpu: int | None) -> tuple[int, int]:
    """(workers, workers per GPU).  Oracle tasks are GPU-bound (no compile
    step unless --compile), so the default is one worker per GPU."""
    if num_gpus <= 0:
        raise ValueError("No matching GPUs found")
    if max_workers is not None and max_workers < 1:
        raise ValueError("--max-workers must be >= 1")
    if workers_per_gpu is not None and workers_per_gpu < 1:
        raise ValueError("--workers-per-gpu must be >= 1")
    if num_tasks <= 0:
        return 0, workers_per_gpu or 1
    if workers_per_gpu is None:
        per_gpu = 1 if max_workers is None else max(1, -(-max_workers // num_gpus))
    else:
        per_gpu = workers_per_gpu
    capacity = num_gpus * per_gpu
    want = max_workers if max_workers is not None else capacity
    return min(want, capacity, num_tasks), per_gpu


# ---------------------------------------------------------------------------
# Worker subprocess (reference :2943-3131)
# ---------------------------------------------------------------------------

def _is_device_error(message: str) -> bool:
    return any(marker in message for marker in _DEVICE_ERROR_MARKERS)


def _bench_oracle_point(canonical_dir: str, shape_label: str, cfg: dict) -> dict:
    """Numerics check of one point, then bench_oracle (or an invalid status)."""
    from oracle_harness import (_load_oracle_module, bench_oracle, check_oracle_all_shapes,
                                get_inputs, get_repro_instance, load_numerics_optout)
    from repro_harness import load_shape_configs, make_inputs_from_config

    _, fn, d = _load_oracle_module(canonical_dir)
    repro_id = d.name
    configs = load_shape_configs(str(d / "repro.py"))
    # The repro's reviewed numerics opt-out applies here as in the runner and
    # bench_oracle_all_shapes (oracle_harness.py:1405-1406, 1848-1888).
    bench_kw = dict(warmup=cfg["n_warmup"], rep=cfg["n_rep"],
                    compare_compile=cfg["compile"],
                    numerics_optout=load_numerics_optout(d))
    if shape_label == _DEFAULT_SHAPE_TOKEN or not configs:
        passed = True
        if not cfg["skip_check"]:
            check = check_oracle_all_shapes(fn, d, repro_id, skip_stochastic=True)
            passed = all(v not in ("fail", False) for v in check.values())
        if not passed:
            return {"default": {"repro_id": repro_id, "status": "UNVERIFIED_NUMERICS"}}
        return {"default": bench_oracle(fn, get_repro_instance(d), get_inputs(d), repro_id,
                                        **bench_kw)}
    if shape_label not in configs:
        return {shape_label: {"repro_id": f"{repro_id}_{shape_label}",
                              "status": "NO_ORACLE_FOR_SHAPE"}}
    point_id = f"{repro_id}_{shape_label}"
    # A point that no registration matches (a withdrawn point of a dir with
    # no shape-general entry) is NO_ORACLE_FOR_SHAPE, bench_oracle's own
    # status for a dispatch miss; the reference's runner reaches it through
    # the failed check instead and reports UNVERIFIED_NUMERICS
    # (scripts/bench_parallel.py:3041-3052).
    from oracle_harness import OracleDispatchError, resolve_oracle
    try:
        resolve_oracle(fn, make_inputs_from_config(configs[shape_label], device="meta"))
    except OracleDispatchError as e:
        return {shape_label: {"repro_id": point_id, "status": "NO_ORACLE_FOR_SHAPE",
                              "error": str(e)[:300]}}
    if not cfg["skip_check"]:
        check = check_oracle_all_shapes(fn, d, repro_id, skip_stochastic=True,
                                        point=shape_label)
        if not all(v not in ("fail", False) for v in check.values()):
            return {shape_label: {"repro_id": point_id, "status": "UNVERIFIED_NUMERICS"}}
    inputs = make_inputs_from_config(configs[shape_label])
    return {shape_label: bench_oracle(fn, get_repro_instance(d), inputs, point_id, **bench_kw)}


def _worker_main(cfg: dict) -> int:
    """Loop: one task key per stdin line -> one JSON line on the result fd.

    fd 1 is pointed at stderr before any work so prints from the harness or
    native libraries cannot corrupt the result pipe (a private dup of the
    original stdout carries the results).  `EXIT` ends the loop; `PREFETCH:`
    lines are accepted and ignored (module loading is cheap here).
    """
    result_file = os.fdopen(os.dup(1), "w", buffering=1)
    os.dup2(2, 1)
    sys.stdout = sys.stderr
    import torch  # noqa: F401  (device initialisation in this process)

    for line in sys.stdin:
        line = line.strip()
        if not line or line == "EXIT":
            break
        if line.startswith("PREFETCH:"):
            continue
        try:
            canonical_dir, label = _split_shape_task_key(line)
            results = _bench_oracle_point(canonical_dir, label or _DEFAULT_SHAPE_TOKEN, cfg)
            results["_repro"] = line
            result_file.write(json.dumps(results, default=str) + "\n")
        except Exception as exc:
            message = str(exc)
            if _is_device_error(message):
                result_file.write(f"DEVICE_ERROR: {message[:1000]}\n")
                result_file.flush()
                return 1
            result_file.write(json.dumps({"_repro": line, "__error__": {
                "status": "failed", "category": "runtime_error",
                "exception_type": type(exc).__name__, "error": message[:1000],
                "reason": "oracle worker failed while benchmarking the point",
                "hint": "Run `python -m oracle_harness <dir> --bench` directly."}}) + "\n")
        result_file.flush()
    return 0


def worker_command(cfg: dict) -> list[str]:
    return [sys.executable, "-u", "-m", "bench_parallel", "--worker", json.dumps(cfg)]


# ---------------------------------------------------------------------------
# Parent side: one thread per worker (reference :2688-2940)
# ---------------------------------------------------------------------------

def _worker_env(gpu_index: str) -> dict:
    from gpu_lock import child_env_for_gpu
    env = child_env_for_gpu(gpu_index)
    env["INDUCTOR_GPU_BENCH_LOCK"] = "1"
    path = [str(PKG_DIR), str(REPO_ROOT)]
    if env.get("PYTHONPATH"):
        path.append(env["PYTHONPATH"])
    env["PYTHONPATH"] = os.pathsep.join(path)
    return env


def _run_worker(gpu: dict, task_queue: "queue.Queue", result_queue: "queue.Queue",
                command: list[str], env: dict | None = None,
                task_timeout_s: float | None = None) -> None:
    """Feed tasks to a persistent worker on `gpu`; respawn it after a device
    error, a death or a misaligned result; every task yields one result."""
    env = _worker_env(gpu["index"]) if env is None else env
    proc = None
    tail: collections.deque = collections.deque(maxlen=20)
    drainer: threading.Thread | None = None

    def spawn():
        nonlocal tail, drainer
        tail = collections.deque(maxlen=20)
        p = subprocess.Popen(command, stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                             stderr=subprocess.PIPE, text=True, bufsize=1, env=env,
                             cwd=str(PKG_DIR))

        def drain(stream, sink):
            for ln in stream:
                if ln.strip():
                    sink.append(ln.rstrip())
        drainer = threading.Thread(target=drain, args=(p.stderr, tail), daemon=True)
        drainer.start()
        return p

    def stop(p):
        if p is None:
            return
        if p.poll() is None:
            try:
                p.stdin.write("EXIT\n")
                p.stdin.flush()
                p.wait(timeout=5)
            except Exception:
                p.kill()
                try:
                    p.wait(timeout=5)
                except Exception:
                    pass
        for s in (p.stdin, p.stdout):
            try:
                s.close()
            except Exception:
                pass

    def stderr_summary():
        # The worker has exited or answered: let the drain thread catch up.
        if drainer is not None and proc is not None and proc.poll() is not None:
            drainer.join(timeout=2)
        lines = list(tail)[-3:]
        return ("; stderr: " + " | ".join(lines)[:300]) if lines else ""

    def fail(task, start, error, **extra):
        result_queue.put({"repro": task, "gpu": gpu["index"], "status": "failed",
                          "elapsed": time.time() - start, "error": error[:1000], **extra})

    while True:
        try:
            task = task_queue.get_nowait()
        except queue.Empty:
            break
        if proc is None or proc.poll() is not None:
            stop(proc)
            proc = spawn()
        start = time.time()
        try:
            proc.stdin.write(task + "\n")
            proc.stdin.flush()
            if task_timeout_s is not None:
                timer = threading.Timer(task_timeout_s, proc.kill)
                timer.start()
            line = proc.stdout.readline()
            if task_timeout_s is not None:
                timer.cancel()
        except Exception as exc:
            stop(proc)
            proc = None
            fail(task, start, str(exc), category="worker_parent_error",
                 exception_type=type(exc).__name__)
            continue
        if not line:
            try:
                code = proc.wait(timeout=5)
            except subprocess.TimeoutExpired:
                code = None
            summary = stderr_summary()
            stop(proc)
            proc = None
            fail(task, start, f"worker exited without a result (returncode={code})" + summary)
            continue
        line = line.strip()
        if line.startswith("{"):
            payload = json.loads(line)
            got = payload.pop("_repro", None)
            if got is not None and got != task:
                stop(proc)
                proc = None
                fail(task, start, f"result misalignment: expected {_task_display_name(task)} "
                     f"but the worker answered for {_task_display_name(got)}; worker reset")
                continue
            err = payload.pop("__error__", None)
            if err is not None:
                fail(task, start, str(err.get("error", "")),
                     category=err.get("category", "runtime_error"), reason=err.get("reason"),
                     hint=err.get("hint"), exception_type=err.get("exception_type"))
                continue
            result_queue.put({"repro": task, "gpu": gpu["index"], "status": "ok",
                              "elapsed": time.time() - start, "results": payload})
        else:
            summary = ""
            if line.startswith("DEVICE_ERROR"):
                try:
                    proc.wait(timeout=5)
                except subprocess.TimeoutExpired:
                    pass
                summary = stderr_summary()
                stop(proc)
                proc = None
            fail(task, start, line[:200] + summary)
    stop(proc)


def run_tasks(tasks: list[str], gpus: list[dict], n_workers: int, command: list[str],
              *, env_for=None, task_timeout_s: float | None = None,
              on_result=None) -> tuple[dict, dict]:
    """Distribute `tasks` over `n_workers` persistent workers (round-robin
    over `gpus`); returns (results by task, failures by task)."""
    task_queue: queue.Queue = queue.Queue()
    for t in tasks:
        task_queue.put(t)
    result_queue: queue.Queue = queue.Queue()
    threads = []
    for i in range(n_workers):
        gpu = gpus[i % len(gpus)]
        env = env_for(gpu) if env_for is not None else None
        th = threading.Thread(target=_run_worker,
                              args=(gpu, task_queue, result_queue, command, env,
                                    task_timeout_s), daemon=True)
        th.start()
        threads.append(th)
    results: dict = {}
    failures: dict = {}
    received = 0
    while received < len(tasks):
        try:
            r = result_queue.get(timeout=30)
        except queue.Empty:
            if not any(th.is_alive() for th in threads):
                break
            continue
        received += 1
        if r["status"] == "ok":
            results[r["repro"]] = r["results"]
        else:
            failures[r["repro"]] = {k: v for k, v in r.items() if k not in ("repro",)}
        if on_result is not None:
            on_result(r, received, len(tasks))
    for th in threads:
        th.join(timeout=10)
    return results, failures


def _best_valid_us(results: dict) -> float | None:
    from oracle_harness import _INVALID_STATUSES
    best = None
    for _, r in _metric_result_items(results):
        us = r.get("oracle_us")
        if r.get("status") not in _INVALID_STATUSES and isinstance(us, (int, float)):
            best = us if best is None else min(best, us)
    return best


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if argv[:1] == ["--worker"]:
        return _worker_main(json.loads(argv[1]))
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("paths", nargs="*", type=Path)
    ap.add_argument("--oracles", action="store_true",
                    help="benchmark the oracles (the only mode of this backend)")
    ap.add_argument("--gpus", default=None, help="comma-separated GPU indices")
    ap.add_argument("--device-kind", default=None, help="only GPUs of this kind (e.g. MI355X)")
    ap.add_argument("--max-workers", type=int, default=None)
    ap.add_argument("--workers-per-gpu", type=int, default=None)
    ap.add_argument("--n-warmup", type=int, default=25)
    ap.add_argument("--n-rep", type=int, default=100)
    ap.add_argument("--compile", dest="compile", action=argparse.BooleanOptionalAction,
                    default=True, help="time the torch.compile (Inductor) comparator "
                                       "(--no-compile: ORACLE_ONLY)")
    ap.add_argument("--oracle-skip-check", action="store_true")
    ap.add_argument("--output", type=Path, default=None,
                    help="timings file for model_graph_accounting --timings")
    ap.add_argument("--task-timeout", type=float, default=None,
                    help="seconds before a silent worker is killed")
    ap.add_argument("--lock-clocks", action=argparse.BooleanOptionalAction, default=False)
    ap.add_argument("--lock-clocks-mhz", type=int, default=DEFAULT_LOCK_MHZ)
    args = ap.parse_args(argv)
    if not args.oracles:
        ap.error("this backend runs the oracle path only: pass --oracles")
    from gpu_lock import discover_gpus

    paths = args.paths or [PKG_DIR / "repros" / "canonical"]
    dirs = find_oracle_dirs(paths)
    if not dirs:
        print("No oracle.py dirs found.")
        return 0
    tasks = _sort_shape_tasks_big_dirs_first(_expand_oracle_shape_tasks(dirs))
    gpus = _filter_gpus(discover_gpus(), args.gpus)
    if args.device_kind:
        want = args.device_kind.lower()
        gpus = [g for g in gpus if g["kind"].lower() == want or want in g["name"].lower()]
    n_workers, per_gpu = _compute_worker_count(num_tasks=len(tasks), num_gpus=len(gpus),
                                               max_workers=args.max_workers,
                                               workers_per_gpu=args.workers_per_gpu)
    print(f"Benchmarking {len(tasks)} oracle shape-points from {len(dirs)} dirs across "
          f"{n_workers} workers on {len(gpus)} GPUs (sharded per shape)", flush=True)
    print("  GPUs: " + ", ".join(f"{g['index']}:{g['kind']}" for g in gpus), flush=True)
    cfg = {"n_warmup": args.n_warmup, "n_rep": args.n_rep, "compile": args.compile,
           "skip_check": args.oracle_skip_check}
    locked = _lock_gpu_clocks([g["index"] for g in gpus], args.lock_clocks_mhz) \
        if args.lock_clocks else set()

    def report(r, done, total):
        name = _task_display_name(r["repro"])
        if r["status"] == "ok":
            best = _best_valid_us(r["results"])
            metric = f"oracle={best:.1f}us" if best is not None else "no-valid-point"
            print(f"  [{done}/{total}] OK   gpu={r['gpu']}  {r['elapsed']:.1f}s  {metric}  {name}",
                  flush=True)
        else:
            print(f"  [{done}/{total}] FAIL gpu={r['gpu']}  {r['elapsed']:.1f}s  {name}: "
                  f"{r['error'][:80]}", flush=True)

    start = time.time()
    try:
        results, failures = run_tasks(tasks, gpus, n_workers, worker_command(cfg),
                                      task_timeout_s=args.task_timeout, on_result=report)
    finally:
        _reset_gpu_clocks(locked)
    elapsed = time.time() - start
    if args.output:
        timed = _write_oracle_timings_output(args.output, results, failures)
        priced = [k for k in timed if k not in _RESERVED_TOP_LEVEL_KEYS]
        print(f"Wrote {args.output}: {len(priced)} priced dirs, "
              f"{len(timed.get('__failures__', {}))} failed", flush=True)
    print(f"Done: {len(results)} ok, {len(failures)} failed, {elapsed:.1f}s", flush=True)
    return 0 if not failures else 1


if __name__ == "__main__":
    sys.exit(main())
