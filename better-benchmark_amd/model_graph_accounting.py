"""Model-level time projection from per-shape oracle timings.

    python -m model_graph_accounting --timings oracle_timings.json --all
    python -m model_graph_accounting --timings oracle_timings.json --model config4 --json

The `--timings` roll-up of the reference's scripts/model_graph_accounting.py
(:398-750), fed with the MI355X timings file that `bench_parallel --oracles
--output` writes.  For each model it sums, over every fused-partition
occurrence, the oracle time of THAT occurrence's shape (never an averaged
ratio, never one per-dir number for all shapes), and gates the headline:
the projection is a number only when every occurrence is priced.

Occurrence source.  The reference finds occurrences by re-tracing the
model's saved full graphs with the capture pipeline's partitioner
(capture_hook); that corpus-production step is outside this backend.  Here
the occurrences come from the canonical dirs themselves: each shapes.json
point lists the models it occurs in and how often
(`"models": {"<model>": {"occurrences": k}}`), and the point's trailing
label token is its shape hash -- the key `points_by_shape` uses.  A model
then owns k occurrences of (pattern, shape hash) per listed point.

Every occurrence lands in exactly one bucket (reference :413-538):
matched (its own shape has a timed point), fallback (the dir is timed but
not at this shape: the dir's median), or unpriced (no usable number).
"""
from __future__ import annotations

import argparse
import json
import sys
from collections import Counter, defaultdict
from dataclasses import dataclass, field
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CANONICAL_DIR = PKG_DIR / "repros" / "canonical"


@dataclass
class PartitionOccurrence:
    """One occurrence of a fused partition in one model."""
    graph_name: str
    pattern_hash: str
    shape_hash: str
    n_ops: int
    op_counts: dict[str, int]
    origin_ops: list[str]
    input_shapes: list[str]
    max_output_shape: list[int] | None
    has_reduction: bool


@dataclass
class GraphAccounting:
    graph_path: str
    graph_name: str
    occurrences: list[PartitionOccurrence] = field(default_factory=list)
    non_fusible: list = field(default_factory=list)
    errors: list[str] = field(default_factory=list)


@dataclass
class ModelAccounting:
    model_name: str
    model_dir: str
    graphs: list[GraphAccounting] = field(default_factory=list)
    manifest_patterns: list[str] = field(default_factory=list)

    @property
    def all_occurrences(self) -> list[PartitionOccurrence]:
        return [o for g in self.graphs for o in g.occurrences]

    @property
    def all_non_fusible(self) -> list:
        return [op for g in self.graphs for op in g.non_fusible]


# ---------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------

def load_timings(timings_path: Path) -> dict[str, dict]:
    """Canonical dir name -> timing entry; reserved `_`-keys dropped."""
    path = Path(timings_path)
    if not path.exists():
        return {}
    try:
        data = json.loads(path.read_text())
    except (json.JSONDecodeError, OSError):
        return {}
    return {k: v for k, v in data.items() if not k.startswith("_")}


def _meta(d: Path) -> dict:
    try:
        return json.loads((d / "meta.json").read_text())
    except (OSError, json.JSONDecodeError):
        return {}


def build_hash_to_repro(canonical_dir: Path = CANONICAL_DIR) -> dict[str, str]:
    """pattern_hash (meta.json) -> canonical dir name."""
    out = {}
    for d in sorted(p for p in Path(canonical_dir).iterdir() if p.is_dir()):
        phash = _meta(d).get("pattern_hash") or d.name.rsplit("_", 1)[-1]
        out[phash] = d.name
    return out


def _input_shapes(point: dict) -> list[str]:
    shapes = []
    for entry in point.get("inputs", []):
        if isinstance(entry, list) and len(entry) >= 2:
            shapes.append(f"{entry[0]}:{entry[1]}")
    return shapes


def collect_model_occurrences(canonical_dir: Path = CANONICAL_DIR) -> dict[str, ModelAccounting]:
    """model name -> its occurrences, from every dir's shapes.json points."""
    models: dict[str, ModelAccounting] = {}
    for d in sorted(p for p in Path(canonical_dir).iterdir() if p.is_dir()):
        meta = _meta(d)
        phash = meta.get("pattern_hash") or d.name.rsplit("_", 1)[-1]
        try:
            points = json.loads((d / "shapes.json").read_text()).get("points", [])
        except (OSError, json.JSONDecodeError):
            continue
        for point in points:
            shape_hash = str(point.get("shape_hash", ""))
            for model, info in (point.get("models") or {}).items():
                count = int((info or {}).get("occurrences", 1))
                acc = models.setdefault(model, ModelAccounting(model_name=model,
                                                               model_dir=str(canonical_dir)))
                if not acc.graphs:
                    acc.graphs.append(GraphAccounting(graph_path="shapes.json",
                                                      graph_name="shapes.json"))
                for _ in range(count):
                    acc.graphs[0].occurrences.append(PartitionOccurrence(
                        graph_name="shapes.json", pattern_hash=phash, shape_hash=shape_hash,
                        n_ops=int(meta.get("n_ops", 1)),
                        op_counts=dict(Counter(meta.get("origin_ops", []))),
                        origin_ops=list(meta.get("origin_ops", [])),
                        input_shapes=_input_shapes(point), max_output_shape=None,
                        has_reduction=meta.get("kind") == "reduction"))
    return models


# ---------------------------------------------------------------------------
# Roll-up and report (reference :413-750)
# ---------------------------------------------------------------------------

def _rollup_occurrence_timings(timing: dict | None, occs: list[PartitionOccurrence]) -> dict:
    """Sum oracle / compile time over occurrences, each at its own shape.

    matched_occ + fallback_occ + unpriced_occ == total_occ.  A timings entry
    without `points_by_shape` (older files) prices every occurrence at the
    dir's representative number (mode "legacy")."""
    total = len(occs)
    if not timing:
        return {"oracle_us_total": None, "compile_us_total": None, "matched_occ": 0,
                "fallback_occ": 0, "unpriced_occ": total, "total_occ": total,
                "mode": "untimed"}
    rep_o, rep_c = timing.get("oracle_us"), timing.get("compile_us")
    rep_o_ok = isinstance(rep_o, (int, float))
    rep_c_ok = isinstance(rep_c, (int, float))
    by_shape = timing.get("points_by_shape")
    if not isinstance(by_shape, dict):
        if not _rollup_occurrence_timings.warned_legacy:
            print("  [warn] timings lack 'points_by_shape'; pricing every occurrence at the "
                  "dir's representative number", file=sys.stderr)
            _rollup_occurrence_timings.warned_legacy = True
        return {"oracle_us_total": round(rep_o * total, 2) if rep_o_ok else None,
                "compile_us_total": round(rep_c * total, 2) if rep_c_ok else None,
                "matched_occ": 0, "fallback_occ": total if rep_o_ok else 0,
                "unpriced_occ": 0 if rep_o_ok else total, "total_occ": total,
                "mode": "legacy"}
    o_sum = c_sum = 0.0
    have_o = have_c = False
    matched = fallback = unpriced = 0
    for occ in occs:
        point = by_shape.get(occ.shape_hash)
        o_us = point.get("oracle_us") if isinstance(point, dict) else None
        c_us = point.get("compile_us") if isinstance(point, dict) else None
        if isinstance(o_us, (int, float)):
            matched += 1
        elif rep_o_ok:
            o_us = rep_o
            fallback += 1
        else:
            o_us = None
            unpriced += 1
        if not isinstance(c_us, (int, float)):
            c_us = rep_c if rep_c_ok else None
        if isinstance(o_us, (int, float)):
            o_sum += o_us
            have_o = True
        if isinstance(c_us, (int, float)):
            c_sum += c_us
            have_c = True
    mode = ("untimed" if unpriced == total else "per_shape" if matched == total else
            "partial" if matched else "fallback_only")
    return {"oracle_us_total": round(o_sum, 2) if have_o else None,
            "compile_us_total": round(c_sum, 2) if have_c else None,
            "matched_occ": matched, "fallback_occ": fallback, "unpriced_occ": unpriced,
            "total_occ": total, "mode": mode}


_rollup_occurrence_timings.warned_legacy = False


def _pattern_rows(acc: ModelAccounting, hash_to_repro: dict[str, str],
                  timings: dict[str, dict]) -> list[dict]:
    by_hash: dict[str, list[PartitionOccurrence]] = defaultdict(list)
    for occ in acc.all_occurrences:
        by_hash[occ.pattern_hash].append(occ)
    rows = []
    for phash, occs in by_hash.items():
        repro_dir = hash_to_repro.get(phash)
        rep = max(occs, key=lambda o: o.n_ops)
        timing = timings.get(repro_dir) if repro_dir else None
        roll = _rollup_occurrence_timings(timing, occs)
        rows.append({
            "pattern_hash": phash, "repro_dir": repro_dir, "trace_equivalent_repro_dirs": [],
            "occurrences": len(occs), "unique_shape_hashes": len({o.shape_hash for o in occs}),
            "n_ops": rep.n_ops, "kind": "reduction" if rep.has_reduction else "pointwise",
            "op_summary": dict(rep.op_counts),
            "representative_input_shapes": rep.input_shapes,
            "max_output_shape": rep.max_output_shape,
            "oracle_us": timing.get("oracle_us") if timing else None,
            "compile_us": timing.get("compile_us") if timing else None,
            "oracle_us_total": roll["oracle_us_total"],
            "compile_us_total": roll["compile_us_total"],
            "matched_occ": roll["matched_occ"], "fallback_occ": roll["fallback_occ"],
            "unpriced_occ": roll["unpriced_occ"], "total_occ": roll["total_occ"],
            "rollup_mode": roll["mode"],
        })
    rows.sort(key=lambda r: -r["occurrences"])
    return rows


def build_model_report(acc: ModelAccounting, hash_to_repro: dict[str, str],
                       timings: dict[str, dict], opset_to_repros: dict | None = None) -> dict:
    """Coverage-gated projection: `fusible_oracle_us_total` is a number only
    when no occurrence is unpriced; `*_partial` always holds the priced sum."""
    rows = _pattern_rows(acc, hash_to_repro, timings)
    timed = [r for r in rows if r["oracle_us_total"] is not None]
    total_o = round(sum(r["oracle_us_total"] for r in timed), 2)
    total_c = round(sum(r["compile_us_total"] for r in timed
                        if r["compile_us_total"] is not None), 2)
    matched = sum(r["matched_occ"] for r in rows)
    fallback = sum(r["fallback_occ"] for r in rows)
    unpriced = sum(r["unpriced_occ"] for r in rows)
    unpriced_kernels = sorted(
        ({"pattern_hash": r["pattern_hash"], "repro_dir": r["repro_dir"],
          "occurrences": r["occurrences"], "unpriced_occ": r["unpriced_occ"],
          "rollup_mode": r["rollup_mode"]} for r in rows if r["unpriced_occ"] > 0),
        key=lambda k: -k["unpriced_occ"])
    complete = unpriced == 0
    unmatched = [r for r in rows if r["repro_dir"] is None]
    found = {r["pattern_hash"] for r in rows}
    manifest = set(acc.manifest_patterns)
    return {
        "model_name": acc.model_name, "model_dir": acc.model_dir,
        "num_graphs": len(acc.graphs),
        "errors": [e for g in acc.graphs for e in g.errors],
        "total_partition_occurrences": len(acc.all_occurrences),
        "unique_patterns": len(found), "unmatched_patterns": len(unmatched),
        "unmatched_no_trace_equivalent": len(unmatched),
        "total_non_fusible_ops": len(acc.all_non_fusible),
        "projection_complete": complete,
        "fusible_oracle_us_total": total_o if complete else None,
        "fusible_compile_us_total": total_c if complete else None,
        "fusible_oracle_us_total_partial": total_o,
        "fusible_compile_us_total_partial": total_c,
        "fusible_oracle_us_total_is_lower_bound": not complete,
        "priced_occurrences": matched + fallback, "matched_occurrences": matched,
        "fallback_occurrences": fallback, "unpriced_occurrences": unpriced,
        "total_occurrences": sum(r["total_occ"] for r in rows),
        "unpriced_kernels": unpriced_kernels, "timed_patterns": len(timed),
        "shape_matched_occurrences": sum(r["matched_occ"] for r in timed),
        "timed_occurrences": sum(r["total_occ"] for r in timed),
        "manifest": {"patterns": sorted(manifest),
                     "in_manifest_not_found": sorted(manifest - found),
                     "in_manifest_not_found_trace_equivalent": {},
                     "in_manifest_not_found_unexplained": sorted(manifest - found),
                     "found_not_in_manifest": sorted(found - manifest) if manifest else []},
        "patterns": rows, "non_fusible_ops": [],
    }


def format_text_report(report: dict) -> str:
    lines = ["=" * 78, f"MODEL: {report['model_name']}", f"DIR:   {report['model_dir']}",
             "=" * 78,
             f"Occurrence sources: {report['num_graphs']} | partition occurrences: "
             f"{report['total_partition_occurrences']} | unique patterns: "
             f"{report['unique_patterns']} | UNMATCHED: {report['unmatched_patterns']}"]
    if report["projection_complete"]:
        lines.append(f"Fusible time projection (SUM of per-shape us over "
                     f"{report['timed_patterns']} timed patterns): "
                     f"oracle={report['fusible_oracle_us_total']}us "
                     f"compile={report['fusible_compile_us_total']}us")
        lines.append(f"  Per-shape coverage: {report['shape_matched_occurrences']}/"
                     f"{report['timed_occurrences']} occurrences priced at own shape "
                     f"(rest fell back to dir median)")
    else:
        kernels = report["unpriced_kernels"]
        lines.append(f"Fusible time projection: INCOMPLETE -- "
                     f"{report['unpriced_occurrences']}/{report['total_occurrences']} partition "
                     f"occurrences across {len(kernels)} kernel pattern(s) are UNPRICED "
                     f"(untimed); complete floor UNAVAILABLE.")
        lines.append(f"  Lower-bound partial sum (priced occurrences only, NOT a floor): "
                     f"oracle={report['fusible_oracle_us_total_partial']}us "
                     f"compile={report['fusible_compile_us_total_partial']}us")
        if kernels:
            preview = ", ".join(f"{k['repro_dir'] or k['pattern_hash']} x{k['unpriced_occ']}"
                                for k in kernels[:6])
            if len(kernels) > 6:
                preview += f", ... +{len(kernels) - 6} more"
            lines.append(f"  Unpriced kernels: {preview}")
    if report["errors"]:
        lines.append(f"ERRORS: {report['errors']}")
    lines += ["", "Fused partitions:",
              f"  {'pattern_hash':32s} {'occur':>5s} {'shapes':>6s} {'kind':9s} "
              f"{'oracle_us':>9s} {'sum_us':>10s}  mode"]
    for r in report["patterns"]:
        o = f"{r['oracle_us']:.1f}" if r["oracle_us"] is not None else "-"
        t = f"{r['oracle_us_total']:.1f}" if r["oracle_us_total"] is not None else "-"
        lines.append(f"  {r['pattern_hash'][:32]:32s} {r['occurrences']:5d} "
                     f"{r['unique_shape_hashes']:6d} {r['kind']:9s} {o:>9s} {t:>10s}  "
                     f"{r['rollup_mode']}{'' if r['repro_dir'] else '  *** UNMATCHED ***'}")
        shapes = ", ".join(r["representative_input_shapes"][:4])
        lines.append(f"  {'':32s} inputs: {shapes}")
    lines.append("")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--model", "-m", default=None, help="model name filter (substring)")
    ap.add_argument("--all", "-a", action="store_true", help="every model")
    ap.add_argument("--json", action="store_true")
    ap.add_argument("--output", "-o", default=None)
    ap.add_argument("--timings", required=True,
                    help="per-oracle timings JSON written by bench_parallel --oracles --output")
    ap.add_argument("--canonical-dir", type=Path, default=CANONICAL_DIR)
    args = ap.parse_args(argv)
    if not args.model and not args.all:
        ap.error("Specify --model <name> or --all")
    models = collect_model_occurrences(args.canonical_dir)
    names = sorted(models)
    if args.model:
        names = [n for n in names if args.model.lower() in n.lower()]
        if not names:
            print(f"No models matching '{args.model}'", file=sys.stderr)
            return 1
    hash_to_repro = build_hash_to_repro(args.canonical_dir)
    timings = load_timings(Path(args.timings))
    print(f"Loaded {len(timings)} oracle timings, {len(names)} model(s)", file=sys.stderr)
    reports = [build_model_report(models[n], hash_to_repro, timings) for n in names]
    text = (json.dumps(reports[0] if len(reports) == 1 else reports, indent=2) if args.json
            else "\n\n".join(format_text_report(r) for r in reports))
    if args.output:
        Path(args.output).parent.mkdir(parents=True, exist_ok=True)
        Path(args.output).write_text(text + "\n")
    else:
        print(text)
    incomplete = sum(1 for r in reports if not r["projection_complete"])
    print(f"Projection coverage: {len(reports) - incomplete}/{len(reports)} models COMPLETE, "
          f"{incomplete} INCOMPLETE (unpriced kernels)", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
