"""Benchmark of the MI355X oracle path; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]
                    [--no-configs] [--no-cpu] [--copy-calibration MIB]

Headline: BASELINE config 2 (per-channel bias + GELU-tanh, bf16 NCHW ->
NHWC [128,256,56,56]); a step is one oracle_forward over one batch of
inputs already resident in HBM.

Steady-state timing: R rotating input sets (together >= 1 GiB, four times
the 256 MB Infinity Cache) and output buffers rotating the same way (a
buffer is rewritten only after >= 1 GiB of other outputs).  L ~ 64 steps
(cycling through the sets) are captured in one hipGraph, so consecutive
kernels run back to back as in a real pipeline (a separate graph per step
would add the ~8 us idle gap a ROCm graph launch costs); no step finds its
inputs in a cache a previous step warmed.  Exactly K steps are timed
between two device synchronisations (wall clock) and, on the launch
stream, between two hipEvents (device time).

value             = algorithmic bytes per step / (wall time per step)   [GB/s]
roofline.achieved = algorithmic bytes / (device time per step)          [GB/s]
roofline.memcopy_sol_us = the reference's memcopy SOL (fp32 add(src, 1,
                    out=dst) over the same bytes) in the same loop;
         vs_memcopy_sol = memcopy_sol_us / kernel_us (> 1: faster than it)
roofline.flat_copy_us = a non-temporal flat copy (hipo_flat_copy) of the
                    config's read and write bytes in the same loop: the
                    ceiling of the access style; vs_flat_copy = flat_copy_us
                    / kernel_us
configs[].pattern_copy_us = where a flat copy does not share the kernel's
                    access pattern, the copy that does (config 4a: two
                    streams in, two out; config 5: the single-pass
                    BatchNorm's register-held slabs without the exchange),
                    same loop; vs_pattern_copy = pattern_copy_us / steady_us
cpu_baseline      = the eager repro (ATen) on the host CPU, os.cpu_count()
                    threads, warmup 1 + min of 5 runs (the min-of-runs
                    CPU timing of the reference's _do_bench,
                    oracle_harness.py:1718, with fewer runs); the
                    CPU oracle (oracle/hipo_ref.c) time rides along.
configs           = every BASELINE config: the same steady-state loop and
                    flat copy; the compiled repro (torch.compile, Inductor)
                    in that same loop (compile_steady_us, steady_ratio =
                    compile_steady_us / steady_us: the status ratio under
                    sustained streaming); plus oracle_harness.bench_oracle (graph-replay
                    timing after a cache flush, the Inductor comparator, the
                    fp64 numerics gate) with the eager repro timed on the host
                    CPU beside it.
"""
from __future__ import annotations

import argparse
import collections
import contextlib
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "better-benchmark_amd"
for _p in (str(PKG), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

CANONICAL = PKG / "repros" / "canonical"
HEADLINE = "pointwise_bias_gelu_tanh_nhwc"
ALL_CONFIGS = [
    ("1", "mean_lastdim_f32"),
    ("2", "pointwise_bias_gelu_tanh_nhwc"),
    ("3", "amax_sum_scaled_masked_softmax"),
    ("4a", "var_mean_residual_layernorm"),
    ("4b", "mean_rmsnorm"),
    ("5", "var_mean_batchnorm_train_relu"),
]
WORKLOAD = {
    "mean_lastdim_f32": "config1 row mean fp32 [8192,4096]",
    "pointwise_bias_gelu_tanh_nhwc": "config2 bias+gelu_tanh bf16 NCHW->NHWC [128,256,56,56]",
    "amax_sum_scaled_masked_softmax": "config3 scaled causal-masked softmax bf16 [384,1024,1024]",
    "var_mean_residual_layernorm": "config4a residual-add LayerNorm bf16 [16384,4096]",
    "mean_rmsnorm": "config4b RMSNorm bf16 [16384,4096]",
    "var_mean_batchnorm_train_relu": "config5 BatchNorm-train fwd+ReLU fp32 [128,256,56,56]",
}
DTYPE = {
    "mean_lastdim_f32": "f32", "pointwise_bias_gelu_tanh_nhwc": "bf16",
    "amax_sum_scaled_masked_softmax": "bf16", "var_mean_residual_layernorm": "bf16",
    "mean_rmsnorm": "bf16", "var_mean_batchnorm_train_relu": "f32",
}
METRIC = "achieved HBM GB/s and % of 8 TB/s SOL per kernel; µs vs host-CPU eager"
PEAK_GBPS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def pmc_traffic(rid):
    """HBM bytes per launch of the repro's kernel from the committed rocprof
    counter summary (profiles/pmc_traffic.json), or None."""
    path = ROOT / "profiles" / "pmc_traffic.json"
    try:
        entry = json.loads(path.read_text())["kernels"].get(rid)
    except (OSError, ValueError, KeyError):
        return None
    return int(entry["traffic_bytes"]) if entry else None


def _baseline_point(rid):
    from repro_harness import load_shape_configs
    cfgs = load_shape_configs(str(CANONICAL / rid / "repro.py"))
    return next(iter(cfgs.items()))


def _cpu_oracle_call(rid, cpu_inputs, threads):
    import oracle as ref
    if rid == "mean_lastdim_f32":
        return lambda: ref.row_mean(cpu_inputs[0], threads=threads)
    if rid == "pointwise_bias_gelu_tanh_nhwc":
        return lambda: ref.bias_gelu_nchw_to_nhwc(*cpu_inputs, threads=threads)
    if rid == "amax_sum_scaled_masked_softmax":
        return lambda: ref.scaled_masked_softmax(cpu_inputs[0], cpu_inputs[1], 0.125, threads=threads)
    if rid == "var_mean_residual_layernorm":
        return lambda: ref.residual_layernorm(*cpu_inputs, 1e-5, threads=threads)
    if rid == "mean_rmsnorm":
        return lambda: ref.rmsnorm(*cpu_inputs, 1e-5, threads=threads)
    return lambda: ref.batchnorm_train(*cpu_inputs, momentum=0.1, eps=1e-5, threads=threads)


def c_oracle_time(rid, cpu_inputs, budget_s: float = 5.0) -> dict:
    """CPU oracle (oracle/hipo_ref.c, OpenMP, fp64 arithmetic) on the full
    workload: min over repeated runs within ~budget_s (at least 2 runs)."""
    threads = os.cpu_count() or 1
    fn = _cpu_oracle_call(rid, cpu_inputs, threads)
    fn()  # warm (page-in, thread pool)
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return {"us": round(min(times) * 1e6, 1), "threads": threads, "runs": len(times)}


def cpu_baseline(rid, cpu_inputs, nbytes) -> dict:
    """The eager repro on the host CPU (os.cpu_count() threads, warmup 1 + min
    of 5 perf_counter runs: the min-of-runs CPU timing of the reference's
    _do_bench, oracle_harness.py:1718, with fewer runs), expressed in the metric's unit
    over the same algorithmic bytes; the CPU oracle's time rides along."""
    import oracle_harness as oh
    _, _, d = oh._load_oracle_module(CANONICAL / rid)
    eager = oh.time_cpu_eager(oh.get_repro_instance(d), cpu_inputs)
    us = eager["cpu_eager_us"]
    return {"value": round(nbytes / (us * 1e-6) / 1e9, 2), "unit": "GB/s",
            "cores": eager["cpu_threads"], "kind": "port",
            "sample": f"full {WORKLOAD[rid]} workload: the eager Repro (ATen on the CPU), "
                      f"torch.set_num_threads(os.cpu_count()), warmup 1 + min of 5",
            "us": us, "cpu_model": eager["cpu_model"], "cpu_affinity": eager.get("cpu_affinity"),
            "c_oracle": c_oracle_time(rid, cpu_inputs)}


# Steps captured per hipGraph (a multiple of the input sets, at most the
# timed steps): each graph replay leaves the GPU idle for ~8 us on ROCm, so
# longer graphs amortise it (64 steps: ~0.13 us per step); the timed run's
# remainder steps are one more graph.
STEPS_PER_GRAPH = 64


def steady_state(rid, steps, warmup, point=None, compiled=False):
    """Back-to-back steps over rotating input sets (see module docstring);
    `point` picks another shapes.json point of the dir (by shape hash) than
    the BASELINE one.  compiled=True times torch.compile(Repro()) (Inductor,
    coordinate-descent tuning as in bench_oracle's comparator) in the same
    loop instead of the oracle."""
    import torch
    import oracle_harness as oh
    from repro_harness import load_shape_configs, make_inputs_from_config

    dev = torch.device("cuda:0")
    if point is None:
        label, cfg = _baseline_point(rid)
    else:
        label, cfg = next((k, v) for k, v in
                          load_shape_configs(str(CANONICAL / rid / "repro.py")).items()
                          if k == point or k.endswith(f"_{point}"))
    _, fn, d = oh._load_oracle_module(CANONICAL / rid)
    instance = oh.get_repro_instance(d)
    oh._seed_input_generation(1)
    cpu_inputs = make_inputs_from_config(cfg, device="cpu")
    nbytes = oh.effective_bytes(instance, cpu_inputs)
    in_bytes = sum(t.numel() * t.element_size() for t in cpu_inputs if isinstance(t, torch.Tensor))
    sets = min(16, max(2, math.ceil((1 << 30) / max(in_bytes, 1))))
    per_graph = sets * max(1, min(STEPS_PER_GRAPH, steps) // sets)
    tail_steps = steps % per_graph
    input_sets = [[t.to(dev) if isinstance(t, torch.Tensor) else t for t in cpu_inputs]
                  for _ in range(sets)]
    if compiled:
        import importlib
        icfg = importlib.import_module("torch._inductor.config")
        icfg.coordinate_descent_tuning = True
        importlib.import_module("torch._dynamo").reset()
        module = torch.compile(instance)

        def impl(inp):
            with torch.no_grad():
                return module(*inp)
        info = None
    else:
        impl, info = oh.resolve_oracle(fn, input_sets[0])
    log(f"{rid}: {label}, {nbytes} algorithmic bytes/step, {sets} input sets, "
        f"{per_graph} steps per graph{' (torch.compile)' if compiled else ''}")
    in_ptrs = {t.data_ptr() for inp in input_sets for t in inp if isinstance(t, torch.Tensor)}
    out_bytes = 0
    for s in range(sets):
        outs = oh._normalize_outputs(impl(input_sets[s]))
        out_bytes = sum(o.numel() * o.element_size() for o in outs
                        if isinstance(o, torch.Tensor) and o.data_ptr() not in in_ptrs)
    torch.cuda.synchronize()
    # Outputs rotate too: a step's output buffers are reused only after at
    # least 1 GiB of other steps' outputs (4x the Infinity Cache), so no
    # write is absorbed by a cache, while the footprint stays that of a real
    # pipeline.  Within a capture, buffers dropped from `recent` return to
    # the graph's pool and later steps reuse them.
    out_sets = max(2, math.ceil((1 << 30) / max(out_bytes, 1)))
    keep = []
    cycle = torch.cuda.CUDAGraph()
    recent = collections.deque(maxlen=out_sets)
    with torch.cuda.graph(cycle):
        for k in range(per_graph):
            recent.append(impl(input_sets[k % sets]))
    keep.extend(recent)
    tail = None  # the timed run's remainder steps, one graph
    if tail_steps:
        tail = torch.cuda.CUDAGraph()
        recent = collections.deque(maxlen=out_sets)
        with torch.cuda.graph(tail):
            for k in range(tail_steps):
                recent.append(impl(input_sets[k % sets]))
        keep.extend(recent)
    singles = []
    for s in range(sets):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            keep.append(impl(input_sets[s]))
        singles.append(g)
    torch.cuda.synchronize()

    def run(n):
        full, rem = divmod(n, per_graph)
        for _ in range(full):
            cycle.replay()
        if rem and rem == tail_steps:
            tail.replay()
        else:
            for k in range(rem):
                singles[k % sets].replay()

    run(warmup)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with oh._gpu_exclusive_lock(f"bench:{rid}"):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        run(steps)
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    device_s = ev0.elapsed_time(ev1) / 1e3 / steps
    wall_s = wall / steps
    out = {
        "label": label, "nbytes": nbytes, "sets": sets, "steps_per_graph": per_graph,
        "dispatch": info and {"matched": info["matched"], "tuned_on": info["tuned_hardware"]},
        "timed": "torch.compile(Repro())" if compiled else "oracle_forward",
        "ms_per_step": round(wall_s * 1e3, 4),
        "device_us_per_step": round(device_s * 1e6, 2),
        "value": round(nbytes / wall_s / 1e9, 1),
        "achieved": round(nbytes / device_s / 1e9, 1),
    }
    del cycle, tail, singles, keep, input_sets
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out, cpu_inputs


def memcopy_sol_steady(nbytes: int, steps: int = 128) -> float:
    """The reference's memcopy speed-of-light construction
    (repro_harness.py:952-958: an fp32 add(src, 1, out=dst) moving nbytes,
    half read, half written) timed in the steady-state loop (rotating
    buffers >= 1 GiB between reuses, steps in one hipGraph, events on the
    launch stream): device us per step.  It is ATen's elementwise kernel
    with cached stores, not a bound -- a non-temporal copy of the same bytes
    runs ~8 % faster on MI355X."""
    import torch
    import oracle_harness as oh
    n = max(nbytes // 8, 1)
    sets = min(16, max(2, math.ceil((1 << 30) / (4 * n))))
    src = [torch.ones(n, dtype=torch.float32, device="cuda") for _ in range(sets)]
    dst = [torch.empty_like(t) for t in src]
    per_graph = sets * max(1, min(STEPS_PER_GRAPH, steps) // sets)
    for k in range(sets):
        torch.add(src[k], 1, out=dst[k])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for k in range(per_graph):
            torch.add(src[k % sets], 1, out=dst[k % sets])
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with oh._gpu_exclusive_lock("bench:memcopy_sol"):
        ev0.record(stream)
        for _ in range(reps):
            g.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (reps * per_graph)
    del g, src, dst
    torch.cuda.empty_cache()
    return round(us, 2)


def flat_copy_steady(read_bytes: int, write_bytes: int, steps: int = 128) -> float:
    """hipo_flat_copy of read_bytes -> write_bytes (rounded to 1 KiB) in the
    steady-state loop (rotating buffers >= 1 GiB between reuses, steps in one
    hipGraph, events on the launch stream): device us per step.  The ceiling
    of the oracle kernels' access style at a config's bytes."""
    import torch
    import hip_oracles
    import oracle_harness as oh
    rb = max(1024, int(round(read_bytes / 1024)) * 1024)
    wb = max(1024, int(round(write_bytes / 1024)) * 1024)
    sets = min(16, max(2, math.ceil((1 << 30) / min(rb, wb))))
    src = [torch.ones(rb // 4, dtype=torch.float32, device="cuda") for _ in range(sets)]
    dst = [torch.empty(wb // 4, dtype=torch.float32, device="cuda") for _ in range(sets)]
    per_graph = sets * max(1, min(STEPS_PER_GRAPH, steps) // sets)
    for k in range(sets):
        hip_oracles.flat_copy(src[k], dst[k])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for k in range(per_graph):
            hip_oracles.flat_copy(src[k % sets], dst[k % sets])
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with oh._gpu_exclusive_lock("bench:flat_copy"):
        ev0.record(stream)
        for _ in range(reps):
            g.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (reps * per_graph)
    del g, src, dst
    torch.cuda.empty_cache()
    return round(us, 2)


def _steady_callable(fn, sets, steps, label):
    """Device us per call of fn(k) (k = the rotating buffer set), captured
    in one hipGraph of back-to-back calls, events on the launch stream."""
    import torch
    import oracle_harness as oh
    per_graph = sets * max(1, min(STEPS_PER_GRAPH, steps) // sets)
    for k in range(sets):
        fn(k)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for k in range(per_graph):
            fn(k % sets)
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with oh._gpu_exclusive_lock(f"bench:{label}"):
        ev0.record(stream)
        for _ in range(reps):
            g.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / (reps * per_graph)
    del g
    return round(us, 2)


def pattern_copy_steady(rid, cpu_inputs, steps: int = 128):
    """The copy that shares a config's access pattern, where a flat copy does
    not, in the steady-state loop: config 4a, a 2-in / 2-out copy of x and
    residual's bytes (hipo_flat_copy2); config 5, x copied with the
    single-pass BatchNorm kernel's own slabs, rounds and register holding
    but no exchange (hipo_hold_copy_f32).  (name, us) or None."""
    import torch
    import hip_oracles
    if rid == "var_mean_residual_layernorm":
        n = cpu_inputs[0].numel()
        sets = max(2, math.ceil((1 << 30) / (4 * 2 * n)))
        bufs = [[torch.ones(n, dtype=torch.bfloat16, device="cuda") for _ in range(4)]
                for _ in range(sets)]
        us = _steady_callable(lambda k: hip_oracles.flat_copy2(*bufs[k]), sets, steps,
                              "flat_copy2")
        del bufs
        torch.cuda.empty_cache()
        return "2-in/2-out copy (hipo_flat_copy2)", us
    if rid == "var_mean_batchnorm_train_relu":
        x = cpu_inputs[0]
        nb = x.numel() * x.element_size()
        sets = max(2, math.ceil((1 << 30) / (2 * nb)))
        src = [x.to("cuda") for _ in range(sets)]
        dst = [torch.empty_like(t) for t in src]
        us = _steady_callable(lambda k: hip_oracles.hold_copy(src[k], out=dst[k]), sets, steps,
                              "hold_copy")
        del src, dst
        torch.cuda.empty_cache()
        return "hold copy (hipo_hold_copy_f32: the kernel's single-read pattern, no exchange)", us
    return None


def read_write_bytes(cpu_inputs, nbytes):
    """(read, write) split of the algorithmic bytes: every tensor input is
    read once, the rest is written."""
    import torch
    seen, rd = set(), 0
    for t in cpu_inputs:
        if isinstance(t, torch.Tensor) and id(t) not in seen:
            seen.add(id(t))
            rd += t.numel() * t.element_size()
    return rd, max(nbytes - rd, 0)


# Compile comparator budget: per-config torch.compile is skipped once the
# run has spent this long, so the default bench stays within minutes.
COMPILE_BUDGET_S = 420.0


def per_config(want_cpu, steady_steps=64, compare_compile=True, coordinate_descent=True,
               t_start=None):
    import torch
    import oracle_harness as oh
    from repro_harness import make_inputs_from_config
    t_start = t_start or time.perf_counter()
    out = []
    for tag, rid in ALL_CONFIGS:
        label, cfg = _baseline_point(rid)
        log(f"config {tag}: {rid}")
        ss, cpu_inputs = steady_state(rid, steady_steps, 8)
        rd, wr = read_write_bytes(cpu_inputs, ss["nbytes"])
        pattern = pattern_copy_steady(rid, cpu_inputs)
        del cpu_inputs
        compile_steady = None
        if compare_compile:
            try:
                cs, _ = steady_state(rid, steady_steps, 8, compiled=True)
                compile_steady = cs["device_us_per_step"]
            except Exception as e:  # Inductor unavailable: the oracle is still timed
                log(f"config {tag}: compiled steady loop failed: {type(e).__name__}: {e}")
        flat_us = flat_copy_steady(rd, wr)
        memcopy_us = memcopy_sol_steady(ss["nbytes"])
        _, fn, d = oh._load_oracle_module(CANONICAL / rid)
        oh._seed_input_generation(1)
        inputs = make_inputs_from_config(cfg, device="cuda")
        elapsed = time.perf_counter() - t_start
        use_compile = compare_compile and elapsed < COMPILE_BUDGET_S
        log(f"config {tag}: bench_oracle (compile comparator: {use_compile}, "
            f"{elapsed:.0f} s elapsed)")
        # bench_oracle prints its own JSON record per point (the runner's
        # output); stdout carries this script's one line only.
        with contextlib.redirect_stdout(sys.stderr):
            r = oh.bench_oracle(fn, oh.get_repro_instance(d), inputs, f"{rid}_{label}",
                                warmup=10, rep=100, rounds=5, compare_compile=use_compile,
                                coordinate_descent=coordinate_descent, cpu_eager=want_cpu,
                                numerics_optout=oh.load_numerics_optout(d))
        entry = {"config": tag, "repro": rid, "status": r.get("status"),
                 "bytes": r.get("bytes"), "read_bytes": rd, "write_bytes": wr,
                 "steady_us": ss["device_us_per_step"], "steady_gbps": ss["achieved"],
                 "steady_sol_frac": round(ss["achieved"] / PEAK_GBPS, 4),
                 "compile_steady_us": compile_steady,
                 "steady_ratio": (round(compile_steady / ss["device_us_per_step"], 4)
                                  if compile_steady else None),
                 "flat_copy_us": flat_us,
                 "vs_flat_copy": round(flat_us / ss["device_us_per_step"], 4),
                 "memcopy_sol_us": memcopy_us,
                 **({"pattern_copy": pattern[0], "pattern_copy_us": pattern[1],
                     "vs_pattern_copy": round(pattern[1] / ss["device_us_per_step"], 4)}
                    if pattern else {}),
                 "steady_vs_memcopy_sol": round(memcopy_us / ss["device_us_per_step"], 4),
                 "traffic": pmc_traffic(rid),
                 "oracle_us": r.get("oracle_us"), "compile_us": r.get("compile_us"),
                 "ratio": r.get("ratio"),
                 "oracle_launch_us": r.get("oracle_launch_us"),
                 "oracle_median_us": r.get("oracle_median_us"),
                 "clean_cache_sol_frac": r.get("clean_cache_sol_frac")}
        if not use_compile and compare_compile:
            entry["compile_skipped"] = f"time budget ({COMPILE_BUDGET_S:.0f} s) spent"
        for k in ("compile", "compile_error"):
            if k in r:
                entry[k] = r[k]
        if "numerics_optout" in r:
            entry["numerics_optout"] = {"accepted": True,
                                        "reason": r["numerics_optout"]["annotation"]["reason"]}
        gate = r.get("numerics_gate")
        if gate is not None:
            entry["numerics_gate_pass"] = gate.get("pass")
            entry["numerics_gate_comparator"] = gate.get("comparator")
            entry["numerics_gate"] = [
                {k: v for k, v in o.items() if k in ("idx", "err_oracle", "err_compiled",
                                                     "threshold", "pass")}
                for o in gate.get("per_output", [])]
        for k in ("cpu_eager_us", "cpu_threads", "cpu_model"):
            if k in r:
                entry[k] = r[k]
        out.append(entry)
        del inputs
        torch.cuda.empty_cache()
    return out


def copy_calibration(mib: int, reps: int = 20) -> None:
    """Copies of known size, for reading rocprof byte counters: the runtime's
    device copy (dst.copy_(src)) and hipo_flat_copy (16-byte non-temporal
    accesses, the oracle kernels' style), `reps` each over the same buffers."""
    import torch
    import hip_oracles
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    for _ in range(reps):
        hip_oracles.flat_copy(src, dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "bytes_written": n * 4,
                      "reps": reps, "kernels": ["runtime copy", "flat_copy_chunks"]}))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--config", default=HEADLINE, help="repro id of the headline workload")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-compile", action="store_true",
                    help="skip the per-config torch.compile (Inductor) comparator")
    ap.add_argument("--no-coordinate-descent", action="store_true",
                    help="Inductor without coordinate-descent tuning")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path "
              "(each MI355X box here has one GPU). Use --gpus 1.", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs the ROCm device", file=sys.stderr)
        return 2
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0
    import hip_oracles
    hip_oracles.load_library()

    t_start = time.perf_counter()
    rid = args.config
    h, cpu_inputs = steady_state(rid, args.steps, args.warmup)
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE[rid],
        "data": "synthetic (seeded N(mu, sigma) inputs of the BASELINE config)",
        "config": {"workload": WORKLOAD[rid], "repro": rid, "point": h["label"],
                   "bytes_per_step": h["nbytes"], "input_sets": h["sets"],
                   "steps_per_graph": h["steps_per_graph"], "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": h["achieved"], "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(h["achieved"] / PEAK_GBPS, 4),
                     "traffic": pmc_traffic(rid), "kernel_us": h["device_us_per_step"]},
        "cpu_baseline": None,
    }
    # The reference's own SOL yardstick on this box, in the same loop (boxes
    # of the pool differ by 1-3 %); > 1 means faster than that copy.
    sol_us = memcopy_sol_steady(h["nbytes"])
    line["roofline"]["memcopy_sol_us"] = sol_us
    line["roofline"]["vs_memcopy_sol"] = round(sol_us / h["device_us_per_step"], 4)
    rd, wr = read_write_bytes(cpu_inputs, h["nbytes"])
    flat_us = flat_copy_steady(rd, wr)
    line["roofline"]["flat_copy_us"] = flat_us
    line["roofline"]["vs_flat_copy"] = round(flat_us / h["device_us_per_step"], 4)
    if not args.no_cpu:
        log("cpu baseline (eager repro on the host CPU)")
        line["cpu_baseline"] = cpu_baseline(rid, cpu_inputs, h["nbytes"])
    del cpu_inputs
    if not args.no_configs:
        line["configs"] = per_config(not args.no_cpu, compare_compile=not args.no_compile,
                                     coordinate_descent=not args.no_coordinate_descent,
                                     t_start=t_start)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
