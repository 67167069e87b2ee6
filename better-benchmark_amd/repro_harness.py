"""Shape-point loading and input generation for canonical repros.

Counterpart of the reference's repro_harness for the oracle path:
`load_shape_configs` (reference: repro_harness.py:56-88) reads a repro's
sibling shapes.json into {label: {"inputs": [spec, ...]}} and
`make_inputs_from_config` (reference: repro_harness.py:430-569) turns one
config into the repro's positional inputs.

Difference from the reference, on purpose: random inputs are drawn on the
CPU from torch's global CPU generator and then copied to the target
device.  After `torch.manual_seed(s)` the CPU and the GPU therefore see
bit-identical inputs, so the host-CPU eager baseline and the GPU oracle can
be compared on the same data.
"""
from __future__ import annotations

import hashlib
import json
import math
import time
from pathlib import Path

import torch

from input_codec import spec_from_compact, render_signature

__all__ = [
    "load_shape_configs", "make_inputs_from_config", "point_label",
    "shape_hash_of", "benchmark_repro", "memcopy_sol_us",
]


def point_label(point: dict) -> str:
    """`<model>_<shape_hash>` label of a shapes.json point."""
    shape_hash = point.get("shape_hash", "unknown")
    models = point.get("models") or {}
    first = next(iter(models), "")
    short = first.rsplit("/", 1)[-1] if first else ""
    return f"{short}_{shape_hash}" if short else shape_hash


def _is_contiguous(shape, stride) -> bool:
    """torch's row-major contiguity: strides of size-1 dims are free, an
    empty tensor is contiguous."""
    if any(d == 0 for d in shape):
        return True
    expected = 1
    for d, s in zip(reversed(shape), reversed(stride)):
        if d != 1 and s != expected:
            return False
        expected *= d
    return True


def shape_hash_of(entries: list) -> str:
    """8-hex identity of a point, the reference's capture-time shape hash
    (capture_hook.py:759-774 over the placeholder info of :331-336): for every
    tensor input the string "<shape list>:<stride list>:<torch dtype>", the
    stride spelled [] when the tensor is contiguous; the strings sorted,
    JSON-encoded, md5, first 8 hex digits.  Shape-parameter inputs are not
    part of it.  The reference's corpus points reproduce under this function
    (tested on every transcribed shapes.json point)."""
    parts = []
    for e in entries:
        spec = spec_from_compact(e)
        if spec["kind"] != "tensor":
            continue
        shape = [int(d) for d in spec["shape"]]
        stride = spec.get("stride")
        stride = [] if stride is None or _is_contiguous(shape, stride) else [int(s) for s in stride]
        parts.append(f"{shape}:{stride}:torch.{spec['dtype']}")
    return hashlib.md5(json.dumps(sorted(parts)).encode()).hexdigest()[:8]


def load_shape_configs(repro_file: str, symbol_bindings: dict | None = None) -> dict:
    """{label: config} for the repro next to `repro_file` ({} if none)."""
    repro_dir = Path(repro_file).parent
    shapes_json = repro_dir / "shapes.json"
    if not shapes_json.exists():
        if symbol_bindings:
            raise ValueError(f"symbol_bindings given but {repro_dir} has no shapes.json")
        return {}
    return _parse_shapes_json(shapes_json, symbol_bindings=symbol_bindings)


def _parse_shapes_json(path: Path, symbol_bindings: dict | None = None) -> dict:
    data = json.loads(Path(path).read_text())
    symbols = data.get("symbols") or {}
    configs = {}
    for point in data.get("points", []):
        entries = point.get("inputs")
        if entries is None:
            continue
        if symbols or symbol_bindings:
            from input_codec import instantiate_point
            entries = instantiate_point(point, symbols, bindings=symbol_bindings,
                                        guards=data.get("guards"))
        cfg = {"inputs": [spec_from_compact(e) for e in entries],
               "signature": render_signature(entries),
               "shape_hash": point.get("shape_hash")}
        if point.get("alias_group_nbytes"):
            cfg["alias_group_nbytes"] = point["alias_group_nbytes"]
        configs[point_label(point)] = cfg
    return configs


def _storage_numel(shape, stride) -> int:
    if any(int(d) == 0 for d in shape):
        return 0
    return 1 + sum((int(d) - 1) * int(s) for d, s in zip(shape, stride))


def _resolve_device(spec_device: str, override) -> torch.device:
    dev = torch.device(override) if override is not None else torch.device(spec_device)
    if dev.type == "cuda" and not torch.cuda.is_available():
        raise RuntimeError(
            "input spec targets the GPU but torch sees no ROCm device; pass "
            "device='cpu' to make_inputs_from_config for a CPU run")
    return dev


def _generate_cpu(shape, dtype: torch.dtype, gen: dict | None) -> torch.Tensor:
    """Values for a dense CPU tensor of `shape` from the global CPU RNG."""
    kind = (gen or {}).get("kind")
    if dtype in (torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8):
        if kind == "constant":
            return torch.full(shape, int(gen.get("value", 0)), dtype=dtype)
        if kind == "permutation":
            size = gen.get("size")
            n = shape[-1] if shape else 1
            size = int(size) if size is not None else n
            rows = math.prod(shape[:-1]) if len(shape) > 1 else 1
            perms = [torch.randperm(size)[:n] for _ in range(rows)]
            return torch.stack(perms).reshape(shape).to(dtype) if shape else perms[0][0].to(dtype)
        if kind == "offsets":
            hi = max(int(gen.get("high", 1)), 1)
            vals, _ = torch.sort(torch.randint(0, hi, shape, dtype=dtype))
            flat = vals.reshape(-1)
            if flat.numel():
                flat[0] = 0
            return vals
        lo = int(gen.get("low", 0)) if gen else 0
        hi = int(gen.get("high", 100)) if gen else 100
        return torch.randint(lo, max(hi, lo + 1), shape, dtype=dtype)
    if dtype == torch.bool:
        return torch.randint(0, 2, shape, dtype=torch.bool)
    # floating point
    if kind == "index":
        lo, hi = int(gen.get("low", 0)), int(gen.get("high", 100))
        return torch.randint(lo, max(hi, lo + 1), shape, dtype=torch.int64).to(dtype)
    if kind == "normal":
        base = torch.randn(shape, dtype=torch.float32)
        return (base * float(gen["std"]) + float(gen["mean"])).to(dtype)
    if kind == "constf":
        return torch.full(shape, float(gen["value"]), dtype=dtype)
    if kind == "triu_fill":
        if len(shape) != 2:
            raise ValueError("triu_fill needs a 2-D tensor")
        full = torch.full(shape, float(gen["value"]), dtype=torch.float32)
        return torch.triu(full, diagonal=int(gen["diagonal"])).to(dtype)
    if kind not in (None, "randn"):
        raise ValueError(f"unknown generator {gen!r} for {dtype}")
    return torch.randn(shape, dtype=dtype)


def make_inputs_from_config(config: dict, *, device=None) -> list:
    """Positional inputs for one shape config.

    Tensors are generated on the CPU (global torch RNG) and copied to the
    spec's device, or to `device` when given (e.g. "cpu" for a host run).
    On the "meta" device only the layout is built (no values, the RNG is
    not drawn from).  Shape params become lists, symints ints, scalars their
    value.
    """
    group_nbytes = config.get("alias_group_nbytes") or []
    groups: dict[int, torch.Tensor] = {}
    result = []
    for spec in config["inputs"]:
        kind = spec.get("kind", "tensor")
        if kind == "shape":
            result.append(list(spec["dims"]))
            continue
        if kind == "symint":
            result.append(int(spec["value"]))
            continue
        if kind == "scalar":
            result.append(spec["value"])
            continue
        shape = [int(d) for d in spec["shape"]]
        dtype = getattr(torch, spec["dtype"].replace("torch.", ""))
        stride = [int(s) for s in (spec.get("stride") or [])] or None
        dev = _resolve_device(spec.get("device", "cuda"), device)
        if dev.type == "meta" and spec.get("alias_group") is None:
            result.append(torch.empty_strided(shape, stride or _contig(shape), dtype=dtype,
                                              device=dev))
            continue
        if spec.get("alias_group") is not None:
            g = int(spec["alias_group"])
            if g not in groups:
                nbytes = group_nbytes[g] if g < len(group_nbytes) else 0
                if nbytes <= 0:
                    raise ValueError(f"alias_group {g} has no recorded nbytes")
                buf = torch.randint(0, 255, (nbytes,), dtype=torch.uint8)
                groups[g] = buf.to(dev)
            typed = groups[g].view(dtype) if dtype != torch.uint8 else groups[g]
            result.append(typed.as_strided(shape, stride or _contig(shape),
                                           int(spec.get("storage_offset", 0))))
            continue
        if spec.get("exact") and spec.get("data") is not None:
            t = torch.tensor(spec["data"], dtype=dtype).reshape(shape)
            result.append(t.to(dev))
            continue
        gen = spec.get("gen") or spec.get("generator")
        if stride and stride != _contig(shape):
            storage = _generate_cpu([_storage_numel(shape, stride)], dtype,
                                    gen if (gen or {}).get("kind") not in ("triu_fill", "permutation") else None)
            t = storage.to(dev).as_strided(shape, stride)
        else:
            t = _generate_cpu(shape, dtype, gen).to(dev)
        result.append(t)
    return result


def _contig(shape) -> list[int]:
    st, acc = [1] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= max(int(shape[i]), 1)
    return st


def memcopy_sol_us(total_bytes: int, *, device="cuda", reps: int = 50) -> float:
    """Measured copy speed-of-light for `total_bytes` of traffic (µs).

    Same construction as the reference (repro_harness.py:952-958): an
    fp32 `add(src, 1, out=dst)` over total_bytes // 8 elements moves
    total_bytes (half read, half written); min over `reps` event-timed runs.
    """
    from oracle_harness import _gpu_exclusive_lock
    n = max(total_bytes // 8, 1)
    src = torch.empty(n, dtype=torch.float32, device=device).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.add(src, 1, out=dst)
    torch.cuda.synchronize()
    best = math.inf
    with _gpu_exclusive_lock("memcopy_sol"):
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            torch.add(src, 1, out=dst)
            b.record()
            b.synchronize()
            best = min(best, a.elapsed_time(b) * 1000.0)
    return best


def benchmark_repro(repro_file, Repro, make_inputs) -> dict:
    """`python repro.py`: run the eager Repro on its default point.

    Prints one JSON line with the eager wall time and the effective bytes.
    (The reference's version times torch.compile; the compile comparison
    for oracles lives in oracle_harness.bench_oracle.)
    """
    from byte_accounting import count_bytes_effective
    inputs = make_inputs()
    mod = Repro()
    with torch.no_grad():
        mod(*inputs)
        if inputs and isinstance(inputs[0], torch.Tensor) and inputs[0].is_cuda:
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        mod(*inputs)
        if inputs and isinstance(inputs[0], torch.Tensor) and inputs[0].is_cuda:
            torch.cuda.synchronize()
        eager_us = (time.perf_counter() - t0) * 1e6
    result = {"repro": str(Path(repro_file).parent.name),
              "eager_us": round(eager_us, 2),
              "bytes": count_bytes_effective(Repro(), make_inputs())}
    print(json.dumps(result))
    return result
