"""Compact JSON encoding of repro input specs (shapes.json `inputs` entries).

Same format as the reference's codec (reference: input_codec.py:1-25):

    [[128, 256, 56, 56], "f32", {"gen": ["normal", 0.5, 2.0]}]   tensor
    ["S", [8, 1024, 512]]                                          shape param
    ["sc", 0.5]                                                    python scalar
    ["sym", 128]                                                   symint

A tensor entry is [shape, dtype, opts?].  Optional opts keys: "st" stride
(absent = contiguous), "dev" device (absent = "cuda"), "off" storage
offset, "gen" generator [kind, *args] (absent = N(0,1) for floats, small
ints for integer dtypes), "data" exact payload, "alias" alias group, "n"
name, "x" passthrough extras.

Generators understood by repro_harness.make_inputs_from_config:
    ["index", lo, hi]     integer values in [lo, hi) (any dtype)
    ["randint", lo, hi]   integer tensor values in [lo, hi)
    ["perm"(, size)]      permutation(s) of range(size)
    ["offsets", hi]       sorted segment offsets starting at 0
    ["const", v]          integer constant
  added here for the MI355X oracle configs (float inputs the reference's
  generators cannot express):
    ["normal", mu, sigma] float N(mu, sigma^2)
    ["constf", v]         float constant (v may be "inf"/"-inf"/"nan")
    ["triu_fill", d, v]   2-D float: v where col - row >= d, else 0
                          (an additive causal mask for d = 1, v = "-inf")
"""
from __future__ import annotations

import math
from typing import Any

SHORT_DTYPE = {
    "float32": "f32", "float16": "f16", "bfloat16": "bf16", "float64": "f64",
    "int64": "i64", "int32": "i32", "int16": "i16", "int8": "i8",
    "bool": "b8", "uint8": "u8", "uint16": "u16", "uint32": "u32",
    "uint64": "u64", "complex64": "c64", "complex128": "c128",
    "float8_e4m3fn": "f8e4m3fn", "float8_e5m2": "f8e5m2",
}
LONG_DTYPE = {short: long for long, short in SHORT_DTYPE.items()}

# Spec keys encoded structurally; every other key travels in opts["x"].
_STRUCTURAL_KEYS = frozenset({
    "kind", "name", "shape", "dtype", "stride", "device", "storage_offset",
    "generator", "gen", "exact", "data", "alias_group",
})


def _short_dtype(name: str) -> str:
    name = str(name)
    if name.startswith("torch."):
        name = name[len("torch."):]
    return SHORT_DTYPE.get(name, name)


def _long_dtype(name: str) -> str:
    return LONG_DTYPE.get(name, name)


def _contiguous_stride(shape) -> list[int]:
    stride = [1] * len(shape)
    acc = 1
    for i in range(len(shape) - 1, -1, -1):
        stride[i] = acc
        acc *= max(int(shape[i]), 1)
    return stride


def _is_contiguous(shape, stride) -> bool:
    # Size-1 dims may carry any stride without changing the layout.
    expect = _contiguous_stride(shape)
    return all(int(d) == 1 or int(s) == int(e)
               for d, s, e in zip(shape, stride, expect))


def float_value(v) -> float:
    """JSON float payload -> float ("inf", "-inf", "nan" strings allowed)."""
    if isinstance(v, str):
        return float(v)  # float() understands inf/-inf/nan
    return float(v)


def _json_float(v: float):
    v = float(v)
    if math.isfinite(v):
        return v
    return "nan" if math.isnan(v) else ("inf" if v > 0 else "-inf")


def gen_to_compact(gen: dict) -> list | None:
    kind = gen.get("kind")
    if kind in (None, "randn"):
        return None
    if kind == "index":
        return ["index", int(gen.get("low", 0)), int(gen.get("high", 100))]
    if kind == "randint":
        return ["randint", int(gen.get("low", 0)), int(gen.get("high", 2))]
    if kind == "permutation":
        return ["perm"] + ([int(gen["size"])] if gen.get("size") is not None else [])
    if kind == "offsets":
        return ["offsets", int(gen.get("high", 1))]
    if kind == "constant":
        return ["const", gen.get("value", 0)]
    if kind == "normal":
        return ["normal", float(gen.get("mean", 0.0)), float(gen.get("std", 1.0))]
    if kind == "constf":
        return ["constf", _json_float(gen.get("value", 0.0))]
    if kind == "triu_fill":
        return ["triu_fill", int(gen.get("diagonal", 1)),
                _json_float(gen.get("value", float("-inf")))]
    return [kind] + [v for k, v in sorted(gen.items()) if k != "kind"]


def gen_from_compact(c: list) -> dict:
    kind = c[0]
    if kind == "index":
        return {"kind": "index", "low": c[1], "high": c[2]}
    if kind == "randint":
        return {"kind": "randint", "low": c[1], "high": c[2]}
    if kind == "perm":
        return {"kind": "permutation", "size": c[1] if len(c) > 1 else None}
    if kind == "offsets":
        return {"kind": "offsets", "high": c[1]}
    if kind == "const":
        return {"kind": "constant", "value": c[1]}
    if kind == "normal":
        return {"kind": "normal", "mean": float(c[1]), "std": float(c[2])}
    if kind == "constf":
        return {"kind": "constf", "value": float_value(c[1])}
    if kind == "triu_fill":
        return {"kind": "triu_fill", "diagonal": int(c[1]), "value": float_value(c[2])}
    return {"kind": kind}


def compact_from_spec(spec: dict, include_name: bool = False) -> list:
    """Verbose in-memory spec dict -> compact JSON entry (lossless)."""
    kind = spec.get("kind", "tensor")
    if kind == "shape":
        return ["S", list(spec["dims"])]
    if kind == "symint":
        return ["sym", spec.get("value", spec.get("hint", 1))]
    if kind == "scalar":
        return ["sc", spec.get("value")]
    entry: list[Any] = [list(spec["shape"]), _short_dtype(spec["dtype"])]
    opts: dict[str, Any] = {}
    if include_name and spec.get("name"):
        opts["n"] = spec["name"]
    stride = spec.get("stride")
    if stride and not _is_contiguous(spec["shape"], stride):
        opts["st"] = list(stride)
    dev = str(spec.get("device", "cuda"))
    if dev.startswith("cuda"):
        dev = "cuda"  # any accelerator ordinal is "the accelerator"
    if dev != "cuda":
        opts["dev"] = dev
    if spec.get("storage_offset", 0):
        opts["off"] = spec["storage_offset"]
    gen = spec.get("gen") or spec.get("generator")
    if gen:
        cg = gen_to_compact(gen)
        if cg is not None:
            opts["gen"] = cg
    if spec.get("exact") and spec.get("data") is not None:
        opts["data"] = spec["data"]
    if spec.get("alias_group") is not None:
        opts["alias"] = spec["alias_group"]
    extras = {k: v for k, v in spec.items()
              if k not in _STRUCTURAL_KEYS and v is not None}
    if extras:
        opts["x"] = extras
    if opts:
        entry.append(opts)
    return entry


def spec_from_compact(entry: list, name: str | None = None) -> dict:
    """Compact JSON entry -> verbose in-memory spec dict."""
    tag = entry[0] if entry else None
    if tag == "S":
        return {"kind": "shape", "name": name, "dims": list(entry[1])}
    if tag == "sym":
        return {"kind": "symint", "name": name, "value": entry[1]}
    if tag == "sc":
        return {"kind": "scalar", "name": name, "value": entry[1]}
    shape = list(entry[0])
    opts = entry[2] if len(entry) > 2 else {}
    spec: dict[str, Any] = {
        "kind": "tensor",
        "name": name,
        "shape": shape,
        "dtype": _long_dtype(entry[1]),
        "stride": list(opts.get("st", _contiguous_stride(shape))),
        "device": opts.get("dev", "cuda"),
        "storage_offset": opts.get("off", 0),
    }
    if "gen" in opts:
        gen = gen_from_compact(opts["gen"])
        spec["gen"] = gen
        spec["generator"] = gen
    if "data" in opts:
        spec["exact"] = True
        spec["data"] = opts["data"]
    if "alias" in opts:
        spec["alias_group"] = opts["alias"]
    if "n" in opts and name is None:
        spec["name"] = opts["n"]
    spec.update(opts.get("x", {}))
    return spec


def render_T(entry_or_spec) -> str:
    """Human-readable T()/S() rendering of one input (documentation only)."""
    entry = (compact_from_spec(entry_or_spec)
             if isinstance(entry_or_spec, dict) else entry_or_spec)
    if entry[0] == "S":
        return f"S({list(entry[1])})"
    if entry[0] == "sym":
        return f"S([{entry[1]}])"
    if entry[0] == "sc":
        return f"Sc({entry[1]})"
    shape, dtype = list(entry[0]), entry[1]
    opts = entry[2] if len(entry) > 2 else {}
    parts = [f"T({shape}", dtype]
    if "st" in opts:
        parts.append(f"stride={tuple(opts['st'])}")
    g = opts.get("gen")
    if g:
        if g[0] == "index":
            parts.append(f"gen=Index({g[2]}, {g[1]})" if g[1] else f"gen=Index({g[2]})")
        elif g[0] == "perm":
            parts.append("gen=Perm()" if len(g) == 1 else f"gen=Perm({g[1]})")
        else:
            parts.append(f"gen={g[0]}{tuple(g[1:])}")
    return ", ".join(parts) + ")"


def render_signature(entries: list) -> str:
    """T()/S() signature string of a whole point, e.g. "(T([8, 4], f32),)"."""
    rendered = [render_T(e) for e in entries]
    return "(" + ", ".join(rendered) + ("," if len(rendered) == 1 else "") + ")"


def instantiate_point(point: dict, symbols: dict, bindings: dict | None = None,
                      guards: list | None = None) -> list:
    """Resolve symbolic dims of a point's compact entries to integers.

    A dim may be an int or a symbol name from `symbols`
    ({name: {"hint": int, "range": [lo, hi]}}).  Values come from `bindings`,
    then the point's own "bindings", then the symbol's hint.  Out-of-range
    values raise ValueError.  Guards (strings over the symbols using + - *
    // and comparisons) must all hold.
    """
    values: dict[str, int] = {}
    point_b = point.get("bindings") or {}
    for sym, meta in (symbols or {}).items():
        if bindings and sym in bindings:
            v = int(bindings[sym])
        elif sym in point_b:
            v = int(point_b[sym])
        else:
            v = int(meta.get("hint", 1))
        lo, hi = (meta.get("range") or [None, None])[:2]
        if (lo is not None and v < int(lo)) or (hi is not None and v > int(hi)):
            raise ValueError(f"symbol {sym}={v} outside range [{lo}, {hi}]")
        values[sym] = v
    for g in guards or []:
        if not _eval_guard(g, values):
            raise ValueError(f"guard {g!r} violated by bindings {values}")

    def dim(d):
        if isinstance(d, int):
            return d
        if isinstance(d, str):
            if d in values:
                return values[d]
            return _eval_int_expr(d, values)
        raise TypeError(f"bad dim {d!r}")

    out = []
    for e in point.get("inputs", []):
        if e and e[0] == "S":
            out.append(["S", [dim(d) for d in e[1]]])
        elif e and e[0] == "sym":
            out.append(["sym", dim(e[1])])
        elif e and e[0] == "sc":
            out.append(list(e))
        else:
            new = [[dim(d) for d in e[0]], e[1]]
            if len(e) > 2:
                opts = dict(e[2])
                if "st" in opts:
                    opts["st"] = [dim(d) for d in opts["st"]]
                new.append(opts)
            out.append(new)
    return out


def _eval_int_expr(expr: str, values: dict) -> int:
    import ast
    import operator
    ops = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul,
           ast.FloorDiv: operator.floordiv, ast.Mod: operator.mod}

    def ev(node):
        if isinstance(node, ast.Expression):
            return ev(node.body)
        if isinstance(node, ast.Constant) and isinstance(node.value, int):
            return node.value
        if isinstance(node, ast.Name) and node.id in values:
            return values[node.id]
        if isinstance(node, ast.BinOp) and type(node.op) in ops:
            return ops[type(node.op)](ev(node.left), ev(node.right))
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub):
            return -ev(node.operand)
        raise ValueError(f"unsupported expression {expr!r}")
    return int(ev(ast.parse(expr, mode="eval")))


def _eval_guard(expr: str, values: dict) -> bool:
    import re
    m = re.fullmatch(r"\s*(.+?)\s*(==|!=|<=|>=|<|>)\s*(.+?)\s*", expr)
    if not m:
        raise ValueError(f"unsupported guard {expr!r}")
    a, op, b = _eval_int_expr(m.group(1), values), m.group(2), _eval_int_expr(m.group(3), values)
    return {"==": a == b, "!=": a != b, "<=": a <= b, ">=": a >= b,
            "<": a < b, ">": a > b}[op]
