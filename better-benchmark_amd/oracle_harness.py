"""Oracle API for MI355X: registration/dispatch, correctness check, ROCm
timing path, fp64 numerics gate, GPU lock, runner CLI.

Public surface (same names, arguments and behaviour as the reference's
oracle_harness.py, whose line numbers are cited per function):

  get_hardware_info, get_shape_key, get_gpu_kind
  OracleRegistry, OracleDispatchError, parse_shapes_signature, oracle_impl,
  get_module_registry, resolve_oracle, reset_oracle_registry
  load_repro_module, get_inputs, get_repro_instance
  has_stochastic_ops, detect_stochastic_outputs
  load_numerics_optout, numerics_optout_applies
  check_oracle, check_oracle_all_shapes
  bench_oracle, bench_oracle_all_shapes
  python -m oracle_harness <repro_dir> [--check|--bench|--bench-unchecked]

What is new for ROCm:
  * get_gpu_kind() reads the HIP device name / gcnArchName ("gfx950" ->
    "MI355X") instead of running nvidia-smi.
  * bench_oracle() times hipGraph replays (torch.cuda.CUDAGraph is a
    hipGraph on ROCm) with a hipEvent pair per replay, and reads a 1 GiB
    buffer between replays, outside the event pair, so inputs never come
    from the 256 MB Infinity Cache.  It reports effective bytes, GB/s and
    the fraction of the MI355X HBM peak next to µs, and can time the eager
    repro on the host CPU in the same call.
  * The torch.compile comparator is optional: when Inductor cannot run,
    the oracle is still timed and gated against eager.
  * The GPU lock also honours HIP_VISIBLE_DEVICES / ROCR_VISIBLE_DEVICES.
"""
from __future__ import annotations

import contextlib
import copy
import fcntl
import importlib.util
import json
import math
import os
import re
import sys
import tempfile
import threading
import time
import warnings
from pathlib import Path

import torch

if __name__ == "__main__":
    sys.modules.setdefault("oracle_harness", sys.modules[__name__])

# ---------------------------------------------------------------------------
# Hardware and shape utilities
# ---------------------------------------------------------------------------

#: HIP arch -> hardware kind when the marketing name is not recognised.
_ARCH_KIND = {"gfx950": "MI355X", "gfx942": "MI300X", "gfx90a": "MI250X"}
_NAME_KINDS = ("MI355X", "MI350X", "MI325X", "MI300X", "MI300A", "MI250X", "MI210")


def get_hardware_info():
    """Device properties for launch-config selection (reference :46-56)."""
    props = torch.cuda.get_device_properties(0)
    return {
        "name": props.name,
        "arch": getattr(props, "gcnArchName", ""),
        "num_cus": props.multi_processor_count,
        "num_sms": props.multi_processor_count,
        "shared_mem_per_sm": getattr(props, "max_shared_memory_per_multiprocessor", None),
        "total_mem_gb": props.total_memory / 1e9,
    }


def get_shape_key(inputs):
    """Tuple of the tensor inputs' shapes (reference :59-65)."""
    return tuple(tuple(t.shape) for t in inputs if isinstance(t, torch.Tensor))


def get_gpu_kind() -> str:
    """Short hardware kind of device 0, e.g. "MI355X"; cached (reference :72-93).

    Tests may force it by setting get_gpu_kind._cached.
    """
    if not hasattr(get_gpu_kind, "_cached"):
        kind = "unknown"
        try:
            if torch.cuda.is_available():
                props = torch.cuda.get_device_properties(0)
                name = props.name or ""
                arch = (getattr(props, "gcnArchName", "") or "").split(":")[0]
                kind = next((k for k in _NAME_KINDS if k in name.replace(" ", "")), None) \
                    or _ARCH_KIND.get(arch) or (name.replace(" ", "_")[:20] or "unknown")
        except Exception:
            kind = "unknown"
        get_gpu_kind._cached = kind
    return get_gpu_kind._cached


# ---------------------------------------------------------------------------
# Registry and dispatch
# ---------------------------------------------------------------------------

_DTYPE_TOKEN = {
    torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16",
    torch.float64: "f64", torch.int64: "i64", torch.int32: "i32",
    torch.int16: "i16", torch.int8: "i8", torch.bool: "b8", torch.uint8: "u8",
}
for _n, _tok in (("float8_e4m3fn", "f8e4m3fn"), ("float8_e5m2", "f8e5m2"),
                 ("float8_e4m3fnuz", "f8e4m3fnuz"), ("float8_e5m2fnuz", "f8e5m2fnuz")):
    if hasattr(torch, _n):
        _DTYPE_TOKEN[getattr(torch, _n)] = _tok


class OracleRegistry:
    """Per-module list of (hardware, shape, configs) implementations.

    Matching is exact-only (reference :151-348): an entry either declares the
    concrete shapes it was written for or is shape-general (shape=None).
    Match order: "hardware+shape" > "shape" > "hardware" > "any"; nothing
    matching raises.  `configs` are passed to the implementation as kwargs.
    """

    def __init__(self):
        self._entries: list[dict] = []
        self.last_dispatch_info = None

    def register(self, hardware=None, shape=None, configs=None, description=None):
        if callable(shape):
            raise TypeError("shape must be a concrete tuple (key input shape) or a "
                            "tuple of tuples (all input shapes), not a predicate")
        norm, full = self._normalize_shape(shape)
        if configs is not None and not isinstance(configs, dict):
            raise TypeError(f"configs must be a dict or None, got {type(configs).__name__}")

        def decorator(fn):
            for prev in self._entries:
                if prev["hardware"] == hardware and prev["shape"] == norm:
                    print(f"WARNING: duplicate oracle registration for (hardware="
                          f"{hardware!r}, shape={norm!r}): {prev['description']} "
                          f"shadows {description or fn.__name__}", file=sys.stderr)
                    break
            self._entries.append({
                "hardware": hardware, "shape": norm, "full_sig": full, "fn": fn,
                "configs": dict(configs) if configs else None,
                "description": description or fn.__name__,
            })
            return fn
        return decorator

    @staticmethod
    def _normalize_shape(shape):
        """-> (tuple of shape tuples or None, covers-all-inputs flag)."""
        if shape is None:
            return None, False
        shape = tuple(shape)
        if not shape:
            return (), True
        if all(isinstance(d, int) for d in shape):
            return (shape,), False
        if all(isinstance(s, (tuple, list, torch.Size)) for s in shape):
            return tuple(tuple(s) for s in shape), True
        raise TypeError(f"shape must be a tuple of ints or of tuples, got {shape!r}")

    @staticmethod
    def _signature_matches(entry, actual_shapes) -> bool:
        if entry["shape"] is None:
            return False
        if entry["full_sig"]:
            return tuple(entry["shape"]) == tuple(actual_shapes)
        return bool(actual_shapes) and tuple(entry["shape"][0]) == tuple(actual_shapes[0])

    def select(self, inputs):
        current = get_gpu_kind()
        actual = get_shape_key(inputs)
        tiers = (
            ("hardware+shape", lambda e: self._signature_matches(e, actual) and e["hardware"] == current),
            ("shape", lambda e: self._signature_matches(e, actual)),
            ("hardware", lambda e: e["shape"] is None and e["hardware"] == current),
            ("any", lambda e: e["shape"] is None and e["hardware"] is None),
        )
        chosen = matched = None
        for label, pred in tiers:
            chosen = next((e for e in self._entries if pred(e)), None)
            if chosen is not None:
                matched = label
                break
        if chosen is None:
            self.last_dispatch_info = None
            raise RuntimeError(
                f"No oracle registered for hardware={current!r} shapes={actual!r}. "
                f"Registry has {len(self._entries)} entries: "
                f"{[e['description'] for e in self._entries]}")
        info = {
            "matched": matched,
            "fallback": matched != "hardware+shape",
            "fn_name": chosen["fn"].__name__,
            "description": chosen["description"],
            "tuned_hardware": chosen["hardware"],
            "registered_shape": chosen["shape"],
            "configs": chosen["configs"],
            "current_hardware": current,
            "actual_shapes": actual,
        }
        reg_dtypes = chosen.get("dtypes")
        if reg_dtypes:
            actual_dtypes = tuple(_DTYPE_TOKEN.get(t.dtype, str(t.dtype))
                                  for t in inputs if isinstance(t, torch.Tensor))
            if (len(actual_dtypes) == len(reg_dtypes)
                    and any(r is not None and a != r for a, r in zip(actual_dtypes, reg_dtypes))):
                info["dtypes_differ"] = True
                info["tuned_dtypes"] = reg_dtypes
                info["actual_dtypes"] = actual_dtypes
        self.last_dispatch_info = info
        return chosen, info

    def dispatch(self, inputs):
        entry, _ = self.select(inputs)
        if entry["configs"]:
            return entry["fn"](inputs, **entry["configs"])
        return entry["fn"](inputs)

    def list_entries(self):
        return [{
            "hardware": e["hardware"],
            "shape": e["shape"][0] if (e["shape"] is not None and not e["full_sig"]) else e["shape"],
            "full_signature": e["full_sig"],
            "fn_name": e["fn"].__name__,
            "configs": e["configs"],
            "description": e["description"],
        } for e in self._entries]

    def clear(self):
        self._entries.clear()
        self.last_dispatch_info = None


_module_registries: dict[str, OracleRegistry] = {}


class OracleDispatchError(RuntimeError):
    """No registered oracle implementation matches the runtime inputs."""


_SIG_DTYPES = ("f32", "f16", "bf16", "f64", "i64", "i32", "i16", "i8", "b8", "u8",
               "f8e4m3fn", "f8e5m2", "f8e4m3fnuz", "f8e5m2fnuz")


def parse_shapes_signature(shapes, *, with_dtypes=False):
    """T()/S() signature string -> tuple of tensor shapes (reference :413-465).

    S() entries are shape params and are skipped; dtypes are returned with
    with_dtypes=True (recorded, never matched).  Tuples pass through.
    """
    if shapes is None:
        return (None, None) if with_dtypes else None
    if not isinstance(shapes, str):
        parsed = tuple(tuple(s) for s in shapes)
        return (parsed, None) if with_dtypes else parsed

    def T(shape, dtype=None, *args, **kwargs):
        return ("T", tuple(shape), dtype)

    def S(dims):
        return ("S", tuple(dims))

    ns = {"__builtins__": {}, "T": T, "S": S,
          "Index": lambda high, low=0: None, "Perm": lambda size=None: None}
    ns.update({d: d for d in _SIG_DTYPES})
    value = eval(shapes, ns)  # noqa: S307 - repo-internal signature strings

    def is_entry(x):
        return (isinstance(x, tuple) and len(x) >= 2 and x[0] in ("T", "S")
                and isinstance(x[1], tuple))

    if is_entry(value) or not isinstance(value, tuple):
        value = (value,)
    tensors = [e for e in value if is_entry(e) and e[0] == "T"]
    shape_tuples = tuple(e[1] for e in tensors)
    if with_dtypes:
        return shape_tuples, tuple(e[2] if len(e) > 2 else None for e in tensors)
    return shape_tuples


def oracle_impl(hardware=None, shapes=None, point=None, description=None, **kwargs):
    """Register `fn` as an implementation (reference :468-549).

    point= is a shape_hash of the sibling shapes.json (resolved now; unknown
    hashes raise OracleDispatchError); shapes= is a T()/S() signature; both
    None means shape-general.  Extra kwargs are launch configs passed to
    fn(inputs, **kwargs) at dispatch.  Returns fn unchanged.
    """
    if point is not None and shapes is not None:
        raise ValueError("oracle_impl: pass point= (hash) or shapes=, not both")
    parsed, dtypes = parse_shapes_signature(shapes, with_dtypes=True)

    def decorator(fn):
        reg = _module_registries.setdefault(fn.__module__, OracleRegistry())
        entry_shapes = parsed
        point_dtypes = dtypes
        if point is not None:
            import inspect
            mod = inspect.getmodule(fn)
            fpath = Path(getattr(mod, "__file__", None) or inspect.getfile(fn))
            shapes_path = fpath.parent / "shapes.json"
            if not shapes_path.exists():
                raise OracleDispatchError(
                    f"oracle_impl(point={point!r}): no shapes.json next to {fpath}")
            data = json.loads(shapes_path.read_text())
            match = next((p for p in data.get("points", [])
                          if p.get("shape_hash") == point), None)
            if match is None:
                known = [p.get("shape_hash") for p in data.get("points", [])]
                raise OracleDispatchError(
                    f"oracle_impl(point={point!r}): hash not in {shapes_path} "
                    f"(known: {known[:8]}{'...' if len(known) > 8 else ''})")
            from input_codec import SHORT_DTYPE, spec_from_compact
            specs = [spec_from_compact(e) for e in match.get("inputs", [])]
            tensors = [s for s in specs if s.get("kind") == "tensor"]
            entry_shapes = tuple(tuple(s["shape"]) for s in tensors)
            point_dtypes = tuple(SHORT_DTYPE.get(s["dtype"], s["dtype"]) for s in tensors)
        reg.register(hardware=hardware, shape=entry_shapes, configs=kwargs or None,
                     description=description)(fn)
        reg._entries[-1]["dtypes"] = point_dtypes
        reg._entries[-1]["point"] = point
        return fn
    return decorator


def get_module_registry(module_name):
    return _module_registries.get(module_name)


def resolve_oracle(oracle_forward, inputs):
    """(callable with configs bound, dispatch info) (reference :557-577).

    Modules without registrations resolve to (oracle_forward, None).
    """
    reg = _module_registries.get(getattr(oracle_forward, "__module__", None))
    if reg is None or not reg._entries:
        return oracle_forward, None
    try:
        entry, info = reg.select(inputs)
    except RuntimeError as e:
        raise OracleDispatchError(str(e)) from e
    if entry["configs"]:
        fn, cfg = entry["fn"], entry["configs"]
        return (lambda inp: fn(inp, **cfg)), info
    return entry["fn"], info


def reset_oracle_registry(module_name=None):
    if module_name is None:
        _module_registries.clear()
    else:
        _module_registries.pop(module_name, None)


# ---------------------------------------------------------------------------
# Module loading
# ---------------------------------------------------------------------------

def load_repro_module(repro_dir: str | Path):
    """Import <repro_dir>/repro.py under a unique name (reference :592-606)."""
    repro_dir = Path(repro_dir)
    path = repro_dir / "repro.py"
    root = repro_dir.parents[2] if repro_dir.match("repros/canonical/*") else repro_dir.parent
    if str(root) not in sys.path:
        sys.path.insert(0, str(root))
    spec = importlib.util.spec_from_file_location(f"{repro_dir.name}_repro", path)
    if spec is None or spec.loader is None:
        raise RuntimeError(f"Could not load repro module from {path}")
    module = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = module
    spec.loader.exec_module(module)
    return module


def get_inputs(repro_dir: str | Path) -> list:
    mod = load_repro_module(repro_dir)
    if hasattr(mod, "make_inputs"):
        return mod.make_inputs()
    if hasattr(mod, "_default_make_inputs"):
        return mod._default_make_inputs()
    raise RuntimeError("Repro has no make_inputs or _default_make_inputs")


def get_repro_instance(repro_dir: str | Path):
    return load_repro_module(repro_dir).Repro()


# ---------------------------------------------------------------------------
# Stochastic outputs and the reviewed numerics opt-out
# ---------------------------------------------------------------------------

_STOCHASTIC_OPS = [
    "aten.dropout", "aten.bernoulli", "aten.rand", "aten.native_dropout",
    "aten.rrelu", "aten.alpha_dropout", "aten.feature_dropout",
    "aten.feature_alpha_dropout",
]


def has_stochastic_ops(repro_path: str | Path) -> bool:
    text = Path(repro_path).read_text()
    return any(op in text for op in _STOCHASTIC_OPS)


#: A gate violation larger than this fraction of the reference's abs-max is
#: not precision drift, and a verified opt-out is refused (reference :688).
NUMERICS_OPTOUT_MAX_REL_DIFF = 0.05
#: Absolute floor of that bound (reference :692).
NUMERICS_OPTOUT_ABS_FLOOR = 1e-2


def load_numerics_optout(repro_dir: str | Path) -> dict | None:
    """The verified `numerics_optout` object of <repro_dir>/meta.json, else None.

    Only {"verified": true, "reason": <non-empty str>, ...} counts; anything
    malformed is treated as absent (reference :695-723).
    """
    meta_path = Path(repro_dir) / "meta.json"
    if not meta_path.exists():
        return None
    try:
        meta = json.loads(meta_path.read_text())
    except (OSError, ValueError):
        return None
    opt = meta.get("numerics_optout") if isinstance(meta, dict) else None
    if not isinstance(opt, dict) or opt.get("verified") is not True:
        return None
    reason = opt.get("reason")
    if not (isinstance(reason, str) and reason.strip()):
        print(f"  NUMERICS_OPTOUT_IGNORED: {meta_path} has a verified opt-out "
              f"without a non-empty 'reason'", file=sys.stderr)
        return None
    return opt


def numerics_optout_applies(numerics_result, optout) -> dict:
    """May a verified opt-out accept this failing gate? (reference :726-804)

    Accepts only if every failing output's error is finite and within
    max(NUMERICS_OPTOUT_MAX_REL_DIFF * ref_absmax, NUMERICS_OPTOUT_ABS_FLOOR).
    """
    if not optout:
        return {"accept": False, "reason": "no verified opt-out"}
    if numerics_result is None:
        return {"accept": False, "reason": "no numerics gate result to accept"}
    offenders, failing = [], 0
    for entry in numerics_result.get("per_output", []):
        if entry.get("pass") is not False:
            continue
        failing += 1
        err = entry.get("err_oracle")
        absmax = entry.get("ref_absmax", 0.0) or 0.0
        if not isinstance(err, (int, float)):
            continue
        if not math.isfinite(err):
            offenders.append({"idx": entry.get("idx"), "err_oracle": err,
                              "ref_absmax": absmax, "plausible_bound": None,
                              "non_finite": True})
            continue
        bound = max(NUMERICS_OPTOUT_MAX_REL_DIFF * max(absmax, 1e-12),
                    NUMERICS_OPTOUT_ABS_FLOOR)
        if err > bound:
            offenders.append({"idx": entry.get("idx"), "err_oracle": err,
                              "ref_absmax": absmax, "plausible_bound": bound})
    if offenders:
        def badness(e):
            v = e["err_oracle"]
            return v if isinstance(v, (int, float)) and math.isfinite(v) else math.inf
        worst = max(offenders, key=badness)
        if worst.get("non_finite"):
            why = (f"output {worst['idx']} diff is non-finite ({worst['err_oracle']}) "
                   f"-- divergence/NaN, not rounding")
        else:
            why = (f"output {worst['idx']} diff {worst['err_oracle']:.3e} exceeds "
                   f"plausible precision-drift bound {worst['plausible_bound']:.3e} "
                   f"(ref_absmax={worst['ref_absmax']:.3e}) -- looks like a real bug")
        return {"accept": False, "reason": f"opt-out REFUSED: {why}", "worst_offender": worst}
    return {"accept": True,
            "reason": f"verified numerics opt-out: {failing} output(s) within "
                      f"plausible precision-drift bound",
            "n_failing": failing}


def detect_stochastic_outputs(instance, inputs) -> set[int]:
    """Indices of outputs that differ between two runs (reference :807-858).

    Each run gets its own copy of the inputs: a repro that updates an input
    in place (BatchNorm running statistics) would otherwise see different
    inputs on the second run and have that output mistaken for a random one
    and skipped by the check.
    """
    def fresh():
        return [_clone_like(t) if isinstance(t, torch.Tensor) else t for t in inputs]

    torch.manual_seed(42)
    if torch.cuda.is_available():
        torch.cuda.manual_seed(42)
    with torch.no_grad():
        first = _normalize_outputs(instance(*fresh()))
        second = _normalize_outputs(instance(*fresh()))
    out = set()
    for i, (a, b) in enumerate(zip(first, second)):
        try:
            if a.is_floating_point():
                same = torch.allclose(a.float(), b.float(), atol=1e-6, rtol=0, equal_nan=True)
            else:
                same = torch.equal(a, b)
        except RuntimeError:
            same = False
        if not same:
            out.add(i)
    return out


# ---------------------------------------------------------------------------
# Correctness
# ---------------------------------------------------------------------------

def _compare_oracle_outputs(eager, oracle_out, stochastic, *, atol, rtol) -> bool:
    """Scope + value comparison (reference :865-923)."""
    ref = _normalize_outputs(eager)
    got = _normalize_outputs(oracle_out)
    if len(got) != len(ref):
        print(f"  SCOPE_MISMATCH: oracle produces {len(got)} outputs, eager produces {len(ref)}")
        return False
    ok_all = True
    for i, (e, o) in enumerate(zip(ref, got)):
        if i in stochastic:
            print(f"  output {i}: SKIP (stochastic)")
            continue
        if e.shape != o.shape:
            print(f"  output {i}: SCOPE_MISMATCH shape oracle={list(o.shape)} eager={list(e.shape)}")
            ok_all = False
            continue
        if e.dtype != o.dtype:
            print(f"  output {i}: WARNING dtype mismatch oracle={o.dtype} eager={e.dtype}")
        if o.device != e.device:
            o = o.to(e.device)
        if not e.is_floating_point():
            ok = torch.equal(e, o)
            print(f"  output {i}: {'PASS' if ok else 'FAIL'} (exact, dtype={e.dtype})")
            ok_all &= ok
            continue
        ef, of = e.float(), o.float()
        diff = (ef - of).abs()
        both_nan = torch.isnan(ef) & torch.isnan(of)
        if both_nan.any():
            diff = torch.where(both_nan, torch.zeros_like(diff), diff)
        max_diff = diff.max().item() if diff.numel() else 0.0
        ok = torch.allclose(ef, of, atol=atol, rtol=rtol, equal_nan=True)
        print(f"  output {i}: {'PASS' if ok else 'FAIL'} (shape={list(e.shape)} "
              f"dtype={e.dtype} max_diff={max_diff:.2e})")
        ok_all &= ok
    return ok_all


def _device_fault_messages() -> list[str]:
    """Faults that HIP kernels recorded in device memory since the last check
    (a bounded cross-workgroup wait that timed out leaves NaN outputs behind
    a successful launch).  Reads and clears the words; synchronises.  Empty
    when no kernel library with such words is loaded."""
    mod = sys.modules.get("hip_oracles")
    if mod is None or not hasattr(mod, "device_faults") or not torch.cuda.is_available():
        return []
    return mod.device_faults(clear=True)


def check_oracle(oracle_forward, instance, inputs, *, atol: float = 1e-2,
                 rtol: float = 1e-2, skip_stochastic: bool = True) -> bool:
    """Eager vs oracle on the same inputs (reference :926-963)."""
    try:
        oracle_forward, _ = resolve_oracle(oracle_forward, inputs)
    except OracleDispatchError as e:
        print(f"  NO_ORACLE_FOR_SHAPE: {str(e)[:200]}")
        return False
    stochastic = detect_stochastic_outputs(instance, inputs) if skip_stochastic else set()
    _device_fault_messages()  # start clean: report only this call's faults
    with torch.no_grad():
        eager = instance(*inputs)
        got = oracle_forward(inputs)
    faults = _device_fault_messages()
    if faults:
        print(f"  DEVICE_FAULT: {'; '.join(faults)[:300]}")
        return False
    return _compare_oracle_outputs(eager, got, stochastic, atol=atol, rtol=rtol)


def _seed_input_generation(seed: int) -> None:
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def check_oracle_all_shapes(oracle_forward, repro_dir, repro_id: str, *,
                            skip_stochastic: bool = True, point: str | None = None,
                            atol: float = 1e-2, rtol: float = 1e-2,
                            device=None) -> dict:
    """check at every shapes.json point; eager and oracle get separate but
    identical (seed 1) input sets (reference :972-1050).  `device` overrides
    the spec's device (e.g. "cpu")."""
    from repro_harness import load_shape_configs, make_inputs_from_config
    repro_dir = Path(repro_dir)
    configs = load_shape_configs(str(repro_dir / "repro.py"))
    if point is not None:
        configs = {label: cfg for label, cfg in configs.items()
                   if label == point or label.endswith(f"_{point}")}
        if not configs:
            print(f"  NO_SHAPE_POINT: {point}")
            return {point: False}
    if not configs:
        return {"default": check_oracle(oracle_forward, get_repro_instance(repro_dir),
                                        get_inputs(repro_dir), atol=atol, rtol=rtol,
                                        skip_stochastic=skip_stochastic)}
    results = {}
    for label, cfg in configs.items():
        print(f"Checking {repro_id}_{label}...")
        instance = get_repro_instance(repro_dir)
        _seed_input_generation(0)
        probe = make_inputs_from_config(cfg, device=device)
        stochastic = detect_stochastic_outputs(instance, probe) if skip_stochastic else set()
        del probe
        _seed_input_generation(1)
        eager_inputs = make_inputs_from_config(cfg, device=device)
        _seed_input_generation(1)
        oracle_inputs = make_inputs_from_config(cfg, device=device)
        try:
            selected, _ = resolve_oracle(oracle_forward, oracle_inputs)
        except OracleDispatchError as e:
            print(f"  NO_ORACLE_FOR_SHAPE: {str(e)[:200]}")
            results[label] = False
            continue
        _device_fault_messages()
        with torch.no_grad():
            eager = instance(*eager_inputs)
            got = selected(oracle_inputs)
        faults = _device_fault_messages()
        if faults:
            print(f"  DEVICE_FAULT: {'; '.join(faults)[:300]}")
            results[label] = False
            continue
        results[label] = _compare_oracle_outputs(eager, got, stochastic, atol=atol, rtol=rtol)
    return results


# ---------------------------------------------------------------------------
# Benchmarking (ROCm timing path)
# ---------------------------------------------------------------------------

#: Bytes read between timed replays so no input is served from the 256 MB
#: Infinity Cache (or the 4 MB L2 of any XCD).
DEFAULT_FLUSH_BYTES = 1 << 30


class _CacheFlusher:
    """Reads a large device buffer (a reduction over it) between replays.

    Reading rather than writing leaves clean lines in the caches, so the
    next timed kernel pays no write-back of flush data.
    """

    def __init__(self, nbytes: int, device):
        n = max(nbytes // 4, 1)
        self.buf = torch.ones(n, dtype=torch.float32, device=device)
        self.out = torch.empty((), dtype=torch.float32, device=device)
        self.nbytes = n * 4

    def __call__(self):
        torch.sum(self.buf, dim=0, out=self.out)  # one read pass, no cast


def _time_launches(launch, warmup, rep, *, flush=None):
    """(min µs, median µs) of `rep` event-timed calls of `launch()`.

    Each call sits alone between a hipEvent pair on the current stream;
    `flush()` (if given) runs before each pair, outside it.  The flush keeps
    the GPU busy while the host enqueues the event pair and the launch, so
    the pair brackets the device work and not the host's launch latency.
    """
    for _ in range(warmup):
        launch()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(rep)]
    for start, end in pairs:
        if flush is not None:
            flush()
        start.record()
        launch()
        end.record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) * 1000.0 for s, e in pairs)
    return times[0], times[len(times) // 2]


def _time_graph(graph, warmup, rep, *, flush=None):
    """(min µs, median µs) of `rep` event-timed replays of a captured graph.

    On ROCm a graph launch leaves the GPU idle for several µs before the
    first node runs, and that gap falls inside the event pair; bench_oracle
    therefore also times direct launches (_time_launches).
    """
    return _time_launches(graph.replay, warmup, rep, flush=flush)


def _meta_copy(inputs):
    out = []
    for t in inputs:
        if isinstance(t, torch.Tensor):
            out.append(torch.empty_strided(t.size(), t.stride(), dtype=t.dtype, device="meta"))
        else:
            out.append(t)
    return out


def effective_bytes(instance, inputs) -> int | None:
    """byte_accounting.count_bytes_effective on meta copies (no device work)."""
    from byte_accounting import count_bytes_effective
    try:
        return count_bytes_effective(copy.deepcopy(instance), _meta_copy(inputs))
    except Exception:
        try:
            cloned = [t.clone() if isinstance(t, torch.Tensor) else t for t in inputs]
            return count_bytes_effective(copy.deepcopy(instance), cloned)
        except Exception:
            return None


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cpu_threads() -> int:
    """Threads for the host-CPU eager baseline: os.cpu_count()."""
    return os.cpu_count() or 1


def time_cpu_eager(instance, inputs, *, warmup: int = 1, rep: int = 5,
                   threads: int | None = None) -> dict:
    """Eager repro on the host CPU: warmup, then min of `rep` perf_counter runs
    (the method of the reference's _do_bench CPU path, :1734-1748), on
    `threads` torch threads (default os.cpu_count())."""
    threads = threads or host_cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        cpu_inputs = [t.detach().to("cpu") if isinstance(t, torch.Tensor) else t for t in inputs]
        inst = copy.deepcopy(instance).to("cpu") if isinstance(instance, torch.nn.Module) else instance
        best = math.inf
        with torch.no_grad():
            for i in range(warmup + rep):
                fresh = [t.clone() if isinstance(t, torch.Tensor) else t for t in cpu_inputs]
                t0 = time.perf_counter()
                inst(*fresh)
                dt = (time.perf_counter() - t0) * 1e6
                if i >= warmup:
                    best = min(best, dt)
    finally:
        torch.set_num_threads(prev)
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"cpu_eager_us": round(best, 1), "cpu_threads": threads, "cpu_model": _cpu_model(),
            "cpu_affinity": affinity}


def bench_oracle(oracle_forward, instance, inputs, repro_id: str, *, warmup: int = 25,
                 rep: int = 200, rounds: int = 5, _skip_numerics_gate: bool = False,
                 numerics_optout: dict | None = None, disable_gpu_lock: bool = False,
                 compare_compile: bool = True, coordinate_descent: bool = True,
                 flush_bytes: int = DEFAULT_FLUSH_BYTES,
                 cpu_eager: bool = False, flat_copy_ceiling: bool = False,
                 hardware: str | None = None) -> dict:
    """Time one oracle point on the GPU (reference :1057-1287, ROCm path).

    Steps: resolve dispatch; torch.compile comparator (Inductor, coordinate
    descent on as in the reference) captured in a graph; oracle captured in a
    hipGraph (any graph-related warning during capture ->
    INVALID_CUDAGRAPH_WARNING); fp64-anchored numerics gate against the
    compiled output (GPU eager when there is no compiled comparator); then,
    under the exclusive GPU lock, `rounds` interleaved rounds of `rep`
    hipEvent-timed graph replays of oracle and compiled, a cache flush before
    each.  `oracle_us` / `compile_us` are the min-of-rounds graph-replay
    times, as in the reference (:1225-1241), and the status GOOD / AT_FLOOR /
    BAD_ORACLE at +-5 % (:1243-1255) comes from them; ORACLE_ONLY without a
    comparator.  Also reported: the oracle's direct-launch minimum
    (`oracle_launch_us`, no graph-launch gap inside the event pair), effective
    bytes and, from the direct-launch time, GB/s and the fraction of the HBM
    peak after a read flush (`clean_cache_*`: the Infinity Cache is clean then
    and can absorb part of the writes, so these flatter write-heavy kernels).
    A fault recorded by a kernel (hip_oracles.device_faults) gives
    ORACLE_DEVICE_FAULT.  With `flat_copy_ceiling`, a flat stream copy of
    the point's read and write bytes (hip_oracles.flat_copy: the oracle
    kernels' access style) is timed the same two ways, and `vs_flat_copy`
    (copy time / oracle time, direct launches) says how close the oracle
    runs to what the memory system delivers for that many bytes.
    """
    from byte_accounting import HBM_PEAK_BYTES_PER_S, achieved_gbps, sol_fraction
    dispatch_info = None
    try:
        oracle_forward, dispatch_info = resolve_oracle(oracle_forward, inputs)
    except OracleDispatchError as e:
        result = {"repro_id": repro_id, "status": "NO_ORACLE_FOR_SHAPE", "error": str(e)[:300]}
        print(json.dumps(result))
        return result

    def with_dispatch(result, full=False):
        if dispatch_info is not None:
            d = {"matched": dispatch_info["matched"]}
            if full:
                d.update(tuned_on=dispatch_info["tuned_hardware"],
                         running_on=dispatch_info["current_hardware"],
                         fallback=dispatch_info["fallback"])
                if dispatch_info.get("dtypes_differ"):
                    d.update(dtypes_differ=True,
                             tuned_dtypes=list(dispatch_info["tuned_dtypes"]),
                             actual_dtypes=list(dispatch_info["actual_dtypes"]))
            result["dispatch"] = d
        return result

    def device_fault(where):
        faults = _device_fault_messages()
        if not faults:
            return None
        result = {"repro_id": repro_id, "status": "ORACLE_DEVICE_FAULT", "where": where,
                  "faults": faults[:5]}
        print(json.dumps(with_dispatch(result)))
        return result

    device = _get_device(inputs)
    if device.type != "cuda":
        return _bench_oracle_cpu(oracle_forward, instance, inputs, repro_id,
                                 warmup=warmup, rep=rep)

    hw = hardware or get_gpu_kind()
    nbytes = effective_bytes(instance, inputs)

    compiled = g_compile = None
    compile_error = None
    compile_wall_s = None
    if compare_compile:
        try:
            import importlib
            icfg = importlib.import_module("torch._inductor.config")
            icfg.coordinate_descent_tuning = bool(coordinate_descent)
            # Fresh dynamo state per shape, as the reference (:1143-1146).
            importlib.import_module("torch._dynamo").reset()
            t0 = time.perf_counter()
            compiled = torch.compile(instance)
            with torch.no_grad():
                for _ in range(5):
                    compiled(*inputs)
            torch.cuda.synchronize()
            compile_wall_s = time.perf_counter() - t0
            g_compile, warns = _capture_graph_checked(lambda: compiled(*inputs))
            if warns:
                result = {"repro_id": repro_id, "status": "INVALID_CUDAGRAPH_WARNING",
                          "warning_source": "compiled", "warnings": warns[:5]}
                print(json.dumps(with_dispatch(result)))
                return result
        except Exception as e:  # Inductor unavailable: oracle still timed
            compiled = g_compile = None
            compile_error = f"{type(e).__name__}: {str(e)[:300]}"

    _device_fault_messages()
    with torch.no_grad():
        for _ in range(3):
            oracle_forward(inputs)
    torch.cuda.synchronize()
    bad = device_fault("warmup")
    if bad:
        return bad
    g_oracle, warns = _capture_graph_checked(lambda: oracle_forward(inputs))
    if warns:
        result = {"repro_id": repro_id, "status": "INVALID_CUDAGRAPH_WARNING",
                  "warning_source": "oracle", "warnings": warns[:5]}
        print(json.dumps(with_dispatch(result)))
        return result

    numerics_result = None
    optout_verdict = None
    if not _skip_numerics_gate:
        comparator = compiled if compiled is not None else instance
        numerics_result = _run_anchored_numerics_gate(oracle_forward, instance, comparator, inputs)
        if numerics_result is not None:
            numerics_result["comparator"] = "compiled" if compiled is not None else "eager"
        bad = device_fault("numerics_gate")
        if bad:
            return bad
        if numerics_result is not None and not numerics_result["pass"]:
            verdict = numerics_optout_applies(numerics_result, numerics_optout)
            if verdict["accept"]:
                optout_verdict = verdict
            else:
                result = {"repro_id": repro_id, "status": "NUMERICS_WORSE_THAN_COMPILED",
                          "numerics_gate": numerics_result}
                if numerics_optout:
                    result["numerics_optout_refused"] = verdict
                print(json.dumps(with_dispatch(result), default=str))
                return result

    flush = _CacheFlusher(flush_bytes, device) if flush_bytes else None

    def run_oracle():
        with torch.no_grad():
            oracle_forward(inputs)

    # Adaptive rep count from a quick estimate (reference :1216-1223).
    quick, _ = _time_graph(g_oracle, 3, 10, flush=flush)
    if g_compile is not None:
        quick = min(quick, _time_graph(g_compile, 3, 10, flush=flush)[0])
    if quick < 50:
        rep = max(rep, 500)
    elif quick < 200:
        rep = max(rep, 300)

    best_graph = best_compile_graph = best_launch = math.inf
    medians = []
    with _gpu_exclusive_lock(repro_id, disabled=disable_gpu_lock):
        for _ in range(warmup):
            g_oracle.replay()
            if g_compile is not None:
                g_compile.replay()
        torch.cuda.synchronize()
        # Interleaved rounds, min-of-N (reference :1225-1241).
        for _ in range(rounds):
            g_min, g_med = _time_graph(g_oracle, warmup, rep, flush=flush)
            best_graph = min(best_graph, g_min)
            medians.append(g_med)
            if g_compile is not None:
                best_compile_graph = min(best_compile_graph,
                                         _time_graph(g_compile, warmup, rep, flush=flush)[0])
            best_launch = min(best_launch,
                              _time_launches(run_oracle, warmup, rep, flush=flush)[0])
    bad = device_fault("timing")
    if bad:
        return bad

    if g_compile is not None:
        ratio = best_compile_graph / best_graph if best_graph > 0 else 0.0
        if optout_verdict is not None:
            status = "NUMERICS_OPTOUT_ACCEPTED"
        elif ratio > 1.05:
            status = "GOOD"
        elif ratio < 0.95:
            status = "BAD_ORACLE"
        else:
            status = "AT_FLOOR"
    else:
        ratio = None
        status = "NUMERICS_OPTOUT_ACCEPTED" if optout_verdict is not None else "ORACLE_ONLY"

    result = {
        "repro_id": repro_id,
        "oracle_us": round(best_graph, 2),
        "compile_us": round(best_compile_graph, 2) if g_compile is not None else None,
        "ratio": round(ratio, 3) if ratio is not None else None,
        "status": status,
        "oracle_median_us": round(sorted(medians)[len(medians) // 2], 2),
        "oracle_launch_us": round(best_launch, 2),
        "hardware": hw,
        "bytes": nbytes,
    }
    if nbytes:
        result["clean_cache_gbps"] = round(achieved_gbps(nbytes, best_launch), 1)
        if hw in HBM_PEAK_BYTES_PER_S:
            result["clean_cache_sol_frac"] = round(sol_fraction(nbytes, best_launch, hw), 4)
            result["sol_peak_gbps"] = HBM_PEAK_BYTES_PER_S[hw] / 1e9
    result["timing"] = {"method": "hipevent pair per hipGraph replay, cache-flush read "
                                  "before each; min over rounds (oracle_us, compile_us)",
                        "launch_method": "hipevent pair per direct launch (oracle_launch_us)",
                        "rep": rep, "rounds": rounds,
                        "flush_bytes": flush.nbytes if flush else 0}
    if compare_compile:
        result["compile"] = {"backend": "inductor",
                             "coordinate_descent_tuning": bool(coordinate_descent),
                             "compile_wall_s": (round(compile_wall_s, 1)
                                                if compile_wall_s is not None else None)}
    if compile_error:
        result["compile_error"] = compile_error
    if numerics_result is not None:
        result["numerics_gate"] = numerics_result
    if optout_verdict is not None:
        result["numerics_optout"] = {"accepted": True, "verdict": optout_verdict,
                                     "annotation": numerics_optout}
    if cpu_eager:
        result.update(time_cpu_eager(instance, inputs))
    if flat_copy_ceiling and nbytes:
        with _gpu_exclusive_lock(repro_id, disabled=disable_gpu_lock):
            ceiling = _flat_copy_ceiling(inputs, nbytes, device, warmup, rep, flush)
        result.update(ceiling)
        if best_launch > 0:
            result["vs_flat_copy"] = round(ceiling["flat_copy_launch_us"] / best_launch, 3)
    print(json.dumps(with_dispatch(result, full=True), default=str))
    return result


def _flat_copy_ceiling(inputs, nbytes, device, warmup, rep, flush) -> dict:
    """hipo_flat_copy moving the point's bytes -- every input tensor's bytes
    read, the rest of the effective bytes written, each rounded to 1 KiB --
    timed as the oracle is: direct launches and graph replays, a cache flush
    before each, min over `rep`."""
    import hip_oracles
    seen, rd = set(), 0
    for t in inputs:
        if isinstance(t, torch.Tensor) and id(t) not in seen:
            seen.add(id(t))
            rd += t.numel() * t.element_size()
    wr = max(nbytes - rd, 0)
    rb = max(1024, int(round(rd / 1024)) * 1024)
    wb = max(1024, int(round(wr / 1024)) * 1024)
    src = torch.ones(rb // 4, dtype=torch.float32, device=device)
    dst = torch.empty(wb // 4, dtype=torch.float32, device=device)

    def copy():
        hip_oracles.flat_copy(src, dst)

    launch_us, _ = _time_launches(copy, warmup, rep, flush=flush)
    g, _warns = _capture_graph_checked(copy)
    graph_us, _ = _time_graph(g, warmup, rep, flush=flush)
    del g, src, dst
    return {"flat_copy_read_bytes": rb, "flat_copy_write_bytes": wb,
            "flat_copy_launch_us": round(launch_us, 2), "flat_copy_us": round(graph_us, 2)}


def _bench_oracle_cpu(oracle_forward, instance, inputs, repro_id, *, warmup, rep):
    """CPU-device fallback of bench_oracle: oracle vs eager, perf_counter."""
    with torch.no_grad():
        oracle_us = _do_bench(lambda: oracle_forward(inputs), torch.device("cpu"),
                              warmup=min(warmup, 3), rep=min(rep, 10))
        eager_us = _do_bench(lambda: instance(*inputs), torch.device("cpu"),
                             warmup=min(warmup, 3), rep=min(rep, 10))
    ratio = eager_us / oracle_us if oracle_us > 0 else 0.0
    status = "GOOD" if ratio > 1.05 else ("BAD_ORACLE" if ratio < 0.95 else "AT_FLOOR")
    result = {"repro_id": repro_id, "oracle_us": round(oracle_us, 2),
              "compile_us": round(eager_us, 2), "comparator": "eager_cpu",
              "ratio": round(ratio, 3), "status": status}
    print(json.dumps(result))
    return result


def _clone_like(t: torch.Tensor) -> torch.Tensor:
    if any(s == 0 for s in t.stride()):
        return t.clone()
    out = torch.empty_strided(t.size(), t.stride(), dtype=t.dtype, device=t.device)
    out.copy_(t)
    return out


def _run_anchored_numerics_gate(oracle_forward, instance, compiled, inputs):
    """Oracle and comparator errors vs an fp64 eager reference (reference
    :1314-1385); each run gets its own copy of the inputs."""
    def fresh():
        return [_clone_like(t) if isinstance(t, torch.Tensor) else t for t in inputs]

    stochastic = detect_stochastic_outputs(instance, fresh())
    precision = "f64"
    try:
        ref_mod = copy.deepcopy(instance).double()
        ref_in = [t.double() if isinstance(t, torch.Tensor) and t.is_floating_point() else t
                  for t in fresh()]
        _seed_input_generation(1)
        with torch.no_grad():
            ref = _normalize_outputs(ref_mod(*ref_in))
        del ref_in
    except Exception:
        precision = "f32"
        try:
            _seed_input_generation(1)
            with torch.no_grad():
                ref = _normalize_outputs(instance(*fresh()))
        except Exception:
            return None
    _seed_input_generation(1)
    with torch.no_grad():
        got = _normalize_outputs(oracle_forward(fresh()))
    _seed_input_generation(1)
    with torch.no_grad():
        cmp_out = _normalize_outputs(compiled(*fresh()))
    if len(got) != len(ref) or len(cmp_out) != len(ref):
        return None
    return _anchored_numerics_gate(got, cmp_out, ref, stochastic, ref_precision=precision)


def bench_oracle_all_shapes(oracle_forward, repro_dir, repro_id, **kwargs):
    """bench_oracle at every shapes.json point (reference :1388-1423)."""
    from repro_harness import load_shape_configs, make_inputs_from_config
    repro_dir = Path(repro_dir)
    if "numerics_optout" not in kwargs:
        kwargs["numerics_optout"] = load_numerics_optout(repro_dir)
    configs = load_shape_configs(str(repro_dir / "repro.py"))
    if not configs:
        return [bench_oracle(oracle_forward, get_repro_instance(repro_dir),
                             get_inputs(repro_dir), repro_id, **kwargs)]
    results = []
    for label, cfg in configs.items():
        _seed_input_generation(1)
        inputs = make_inputs_from_config(cfg)
        results.append(bench_oracle(oracle_forward, get_repro_instance(repro_dir), inputs,
                                    f"{repro_id}_{label}", **kwargs))
    return results


# ---------------------------------------------------------------------------
# Graph capture with a warning trap
# ---------------------------------------------------------------------------

def _capture_graph(fn):
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


_CUDAGRAPH_WARNING_PATTERNS = re.compile(
    r"CUDAGraph|cuda.?graph|hip.?graph|graph.?capture|stream.?capture", re.IGNORECASE)


def _capture_graph_checked(fn):
    """(graph, graph-related warning messages); any message invalidates it."""
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        g = _capture_graph(fn)
    msgs = [str(w.message) for w in caught if _CUDAGRAPH_WARNING_PATTERNS.search(str(w.message))]
    return g, msgs


def _anchored_numerics_gate(oracle_outs, compiled_outs, ref_outs, stochastic, *,
                            ref_precision: str = "f64") -> dict:
    """Per float output: pass iff err_oracle <= max(3 err_compiled,
    1e-5 max(|ref|max, 1)), errors = max abs diff vs the fp64 reference
    (reference :1479-1548)."""
    result = {"pass": True, "per_output": [], "worst_output_idx": None,
              "ref_precision": ref_precision}
    worst = 0.0
    for i, (o, c, r) in enumerate(zip(oracle_outs, compiled_outs, ref_outs)):
        entry = {"idx": i}
        if i in stochastic:
            entry["skip"] = "stochastic"
        elif not r.is_floating_point():
            entry["skip"] = "non_float"
        else:
            r64 = r.double()
            err_o = (o.double().to(r64.device) - r64).abs().max().item() if r.numel() else 0.0
            err_c = (c.double().to(r64.device) - r64).abs().max().item() if r.numel() else 0.0
            absmax = r64.abs().max().item() if r.numel() else 0.0
            threshold = max(3.0 * err_c, 1e-5 * max(absmax, 1.0))
            ok = err_o <= threshold
            entry.update(err_oracle=err_o, err_compiled=err_c, threshold=threshold,
                         ref_absmax=absmax, **{"pass": ok})
            if not ok:
                result["pass"] = False
                ratio = err_o / max(err_c, 1e-30)
                if ratio > worst:
                    worst = ratio
                    result["worst_output_idx"] = i
        result["per_output"].append(entry)
    return result


# ---------------------------------------------------------------------------
# Exclusive GPU lock
# ---------------------------------------------------------------------------

_GPU_BENCH_LOCK_STATE_NAME = "_torchinductor_gpu_benchmark_lock_state"


def _env_flag_enabled(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in ("1", "true", "yes", "on")


def _safe_lock_component(value: str) -> str:
    return re.sub(r"[^A-Za-z0-9_.-]+", "_", value.strip()) or "unknown"


def _gpu_bench_lock_state():
    """Process-wide lock state shared by every copy of this module."""
    import builtins
    state = getattr(builtins, _GPU_BENCH_LOCK_STATE_NAME, None)
    if state is None:
        state = {"mutex": threading.RLock(), "local": threading.local()}
        setattr(builtins, _GPU_BENCH_LOCK_STATE_NAME, state)
    return state


def _write_gpu_lock_metadata(fd, gpu, mode, label):
    try:
        os.ftruncate(fd, 0)
        os.write(fd, (f"pid={os.getpid()}\ngpu={gpu}\nmode={mode}\nlabel={label}\n"
                      f"acquired_unix={time.time():.0f}\n").encode())
        os.fsync(fd)
    except OSError:
        pass


def _release_fd(fd):
    if fd is None:
        return
    try:
        fcntl.flock(fd, fcntl.LOCK_UN)
    finally:
        os.close(fd)


def _lock_dir() -> str:
    return (os.environ.get("INDUCTOR_GPU_BENCH_LOCK_DIR")
            or os.environ.get("TORCHINDUCTOR_GPU_BENCH_LOCK_DIR")
            or os.environ.get("COMPILE_UTILS_GPU_LOCK_DIR")
            or os.path.join(tempfile.gettempdir(), "compile_utils_gpu_locks"))


def _lock_gpu_id() -> str:
    """First visible device id; HIP/ROCR visibility lists take precedence."""
    for var in ("HIP_VISIBLE_DEVICES", "ROCR_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES"):
        ids = [d.strip() for d in os.environ.get(var, "").split(",") if d.strip()]
        if ids:
            return _safe_lock_component(ids[0])
    return "0"


@contextlib.contextmanager
def _gpu_exclusive_lock(label="oracle_bench", *, disabled=False):
    """Exclusive per-GPU flock, re-entrant per thread (reference :1614-1692).

    On by default; INDUCTOR_GPU_BENCH_LOCK=1 / TORCHINDUCTOR_GPU_BENCH_LOCK=1
    force it on even when disabled=True.  Takes <dir>/gpu_<id>.gate, then
    <dir>/gpu_<id>.lock, and writes pid/gpu/mode/label metadata.
    """
    forced = (_env_flag_enabled("INDUCTOR_GPU_BENCH_LOCK")
              or _env_flag_enabled("TORCHINDUCTOR_GPU_BENCH_LOCK"))
    if disabled and not forced:
        yield
        return
    lock_dir = _lock_dir()
    os.makedirs(lock_dir, exist_ok=True)
    gpu = _lock_gpu_id()
    lock_path = os.path.join(lock_dir, f"gpu_{gpu}.lock")
    gate_path = os.path.join(lock_dir, f"gpu_{gpu}.gate")
    state = _gpu_bench_lock_state()
    local = state["local"]
    if getattr(local, "depth", 0) > 0 and getattr(local, "mode", None) == "exclusive":
        local.depth += 1
        try:
            yield
        finally:
            local.depth -= 1
        return
    with state["mutex"]:
        fd = gate_fd = None
        try:
            fd = os.open(lock_path, os.O_CREAT | os.O_RDWR, 0o666)
            gate_fd = os.open(gate_path, os.O_CREAT | os.O_RDWR, 0o666)
            fcntl.flock(gate_fd, fcntl.LOCK_EX)
            fcntl.flock(fd, fcntl.LOCK_EX)
            _write_gpu_lock_metadata(fd, gpu, "exclusive", label)
            local.depth, local.mode, local.fd = 1, "exclusive", fd
            try:
                yield
            finally:
                local.depth, local.mode, local.fd = 0, None, None
        finally:
            _release_fd(fd)
            _release_fd(gate_fd)


# ---------------------------------------------------------------------------
# Small helpers
# ---------------------------------------------------------------------------

def _normalize_outputs(out) -> list[torch.Tensor]:
    if isinstance(out, torch.Tensor):
        return [out]
    if isinstance(out, (tuple, list)):
        flat = []
        for item in out:
            if isinstance(item, torch.Tensor):
                flat.append(item)
            elif isinstance(item, (tuple, list)):
                flat.extend(_normalize_outputs(item))
        return flat
    return []


def _get_device(inputs) -> torch.device:
    for t in inputs:
        if isinstance(t, torch.Tensor):
            return t.device
    return torch.device("cuda" if torch.cuda.is_available() else "cpu")


def _do_bench(fn, device: torch.device, warmup: int = 25, rep: int = 200) -> float:
    """min-of-rep wall time of fn() in µs (synchronising on the GPU)."""
    for _ in range(warmup):
        fn()
    if device.type == "cuda":
        torch.cuda.synchronize()
    best = math.inf
    for _ in range(rep):
        t0 = time.perf_counter()
        fn()
        if device.type == "cuda":
            torch.cuda.synchronize()
        best = min(best, (time.perf_counter() - t0) * 1e6)
    return best


# ---------------------------------------------------------------------------
# Runner CLI: python -m oracle_harness <repro_dir> [--check|--bench]
# ---------------------------------------------------------------------------

def _load_oracle_module(canonical_dir):
    d = Path(canonical_dir)
    path = d / "oracle.py"
    if not path.exists():
        candidates = sorted(d.glob("oracle_*.py"))
        if not candidates:
            raise FileNotFoundError(f"no oracle.py / oracle_*.py in {d}")
        path = candidates[0]
    spec = importlib.util.spec_from_file_location(f"_oracle_{d.name}", path)
    reset_oracle_registry(spec.name)  # re-loading must not register twice
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    fn = getattr(mod, "oracle_forward", None)
    if fn is None:
        raise AttributeError(f"{path} defines no oracle_forward")
    return mod, fn, d


_INVALID_STATUSES = frozenset({
    "UNVERIFIED_NUMERICS",
    "INVALID_CUDAGRAPH_WARNING",
    "NUMERICS_WORSE_THAN_COMPILED",
    "NO_ORACLE_FOR_SHAPE",
    # Not in the reference: a kernel recorded a fault (its outputs are NaN).
    "ORACLE_DEVICE_FAULT",
})


def oracle_main(oracle_file, oracle_forward, argv=None) -> int:
    """The standalone CLI of one oracle.py (`python oracle.py [--check]
    [--bench] ...`), the flags of the reference's oracle template
    (scripts/oracle_template.py:147-237): with neither --check nor --bench
    both run; --check compares with the eager Repro on the default inputs
    (every shapes.json point with --all-shapes) and exits 1 on a mismatch;
    --bench times through bench_oracle (locked, graph-captured).  Used as

        if __name__ == "__main__":
            raise SystemExit(oracle_main(__file__, oracle_forward))
    """
    import argparse
    repro_dir = Path(oracle_file).resolve().parent
    repro_id = repro_dir.name
    ap = argparse.ArgumentParser(description=f"Oracle for {repro_id}")
    ap.add_argument("--check", action="store_true", help="verify against the eager Repro")
    ap.add_argument("--bench", action="store_true", help="benchmark the oracle")
    ap.add_argument("--rtol", type=float, default=1e-2)
    ap.add_argument("--atol", type=float, default=1e-2)
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--rep", type=int, default=200)
    ap.add_argument("--no-skip-stochastic", action="store_true")
    ap.add_argument("--all-shapes", action="store_true",
                    help="every shapes.json point instead of the default one")
    ap.add_argument("--disable-gpu-lock", action="store_true")
    ap.add_argument("--no-compile", action="store_true",
                    help="skip the torch.compile comparator (status ORACLE_ONLY)")
    ap.add_argument("--cpu-eager", action="store_true",
                    help="also time the eager repro on the host CPU")
    ap.add_argument("--show-hw", action="store_true", help="print device info and exit")
    ap.add_argument("--device", default=None,
                    help="override the input device of --check (e.g. cpu)")
    args = ap.parse_args(argv)
    if args.show_hw:
        print(json.dumps(get_hardware_info(), indent=2))
        return 0
    if not args.check and not args.bench:
        args.check = args.bench = True
    skip = not args.no_skip_stochastic
    if args.check:
        if args.all_shapes:
            res = check_oracle_all_shapes(oracle_forward, repro_dir, repro_id,
                                          skip_stochastic=skip, atol=args.atol, rtol=args.rtol,
                                          device=args.device)
            ok = not any(v in ("fail", False) for v in res.values())
        else:
            _seed_input_generation(1)
            if args.device is None:
                inputs = get_inputs(repro_dir)
            else:
                from repro_harness import load_shape_configs, make_inputs_from_config
                cfg = next(iter(load_shape_configs(str(repro_dir / "repro.py")).values()))
                inputs = make_inputs_from_config(cfg, device=args.device)
            ok = check_oracle(oracle_forward, get_repro_instance(repro_dir), inputs,
                              atol=args.atol, rtol=args.rtol, skip_stochastic=skip)
        print(f"Correctness: {'PASS' if ok else 'FAIL'}")
        if not ok:
            return 1
    if args.bench:
        kw = dict(warmup=args.warmup, rep=args.rep, disable_gpu_lock=args.disable_gpu_lock,
                  compare_compile=not args.no_compile, cpu_eager=args.cpu_eager,
                  numerics_optout=load_numerics_optout(repro_dir))
        if args.all_shapes:
            results = bench_oracle_all_shapes(oracle_forward, repro_dir, repro_id, **kw)
        else:
            _seed_input_generation(1)
            results = [bench_oracle(oracle_forward, get_repro_instance(repro_dir),
                                    get_inputs(repro_dir), repro_id, **kw)]
        for r in results:
            print(json.dumps(r, default=str))
        if any(isinstance(r, dict) and r.get("status", "") in _INVALID_STATUSES for r in results):
            return 1
    return 0


def _runner_main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(prog="python -m oracle_harness",
                                 description="check/bench runner for oracle.py files")
    ap.add_argument("canonical_dir", help="repros/canonical/<repro_id> directory")
    ap.add_argument("--check", action="store_true",
                    help="numerics check vs Repro() at every shapes.json point")
    ap.add_argument("--no-skip-stochastic", action="store_true")
    ap.add_argument("--bench", action="store_true",
                    help="hipGraph bench at every point (runs --check first and refuses "
                         "to time points whose check failed)")
    ap.add_argument("--bench-unchecked", action="store_true",
                    help="bench without the check gate (results not validated)")
    ap.add_argument("--warmup", type=int, default=25)
    ap.add_argument("--rep", type=int, default=100)
    ap.add_argument("--point", default=None, help="restrict to one shape_hash")
    ap.add_argument("--disable-gpu-lock", action="store_true")
    ap.add_argument("--no-compile", action="store_true",
                    help="skip the torch.compile comparator (status ORACLE_ONLY)")
    ap.add_argument("--cpu-eager", action="store_true",
                    help="also time the eager repro on the host CPU")
    ap.add_argument("--flat-copy", action="store_true",
                    help="also time a flat copy of the point's bytes (vs_flat_copy)")
    ap.add_argument("--device", default=None,
                    help="override the input device for --check (e.g. cpu)")
    args = ap.parse_args(argv)

    mod, fn, d = _load_oracle_module(args.canonical_dir)
    repro_id = d.name
    out = {"repro": repro_id, "oracle": getattr(mod, "__file__", "?")}
    do_bench = args.bench or args.bench_unchecked
    do_check = args.check or (args.bench and not args.bench_unchecked)
    if do_check:
        out["check"] = check_oracle_all_shapes(
            fn, d, repro_id, skip_stochastic=not args.no_skip_stochastic,
            point=args.point, device=args.device)
    if do_bench:
        if args.bench_unchecked:
            print("WARNING: --bench-unchecked bypasses the numerics check gate; results "
                  "are NOT validated.", file=sys.stderr)
        from repro_harness import load_shape_configs, make_inputs_from_config
        configs = load_shape_configs(str(d / "repro.py"))
        if args.point is not None:
            configs = {k: v for k, v in configs.items()
                       if k == args.point or k.endswith(f"_{args.point}")}
        optout = load_numerics_optout(d)
        chk = out.get("check", {})
        kw = dict(warmup=args.warmup, rep=args.rep, numerics_optout=optout,
                  disable_gpu_lock=args.disable_gpu_lock,
                  compare_compile=not args.no_compile, cpu_eager=args.cpu_eager,
                  flat_copy_ceiling=args.flat_copy)
        results = []
        items = list(configs.items()) or [("default", None)]
        for label, cfg in items:
            point_id = repro_id if cfg is None else f"{repro_id}_{label}"
            passed = args.bench_unchecked or not do_check or chk.get(label) not in ("fail", False)
            if not passed:
                results.append({"repro_id": point_id, "status": "UNVERIFIED_NUMERICS"})
                continue
            _seed_input_generation(1)
            inputs = get_inputs(d) if cfg is None else make_inputs_from_config(cfg)
            results.append(bench_oracle(fn, get_repro_instance(d), inputs, point_id, **kw))
        out["bench"] = results
    print(json.dumps(out, indent=1, default=str))
    failed = isinstance(out.get("check"), dict) and any(
        v in ("fail", False) for v in out["check"].values())
    for b in out.get("bench") or []:
        if isinstance(b, dict) and b.get("status", "") in _INVALID_STATUSES:
            failed = True
    return 1 if failed else 0


if __name__ == "__main__":
    raise SystemExit(_runner_main())
