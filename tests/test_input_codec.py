"""input_codec + repro_harness: compact encoding round trips, the float
generators added for the BASELINE inputs, shape hashes, shapes.json loading
and CPU/GPU-identical input generation."""
import json
import math

import pytest
import torch

from input_codec import (compact_from_spec, instantiate_point, render_signature,
                         spec_from_compact)
from repro_harness import (load_shape_configs, make_inputs_from_config, point_label,
                           shape_hash_of)

ENTRIES = [
    [[128, 128, 28, 28], "bf16", {"st": [100352, 1, 3584, 128]}],
    [[4096], "i64", {"gen": ["index", 0, 1000]}],
    [[256], "f32", {"gen": ["normal", 0.5, 2.0]}],
    [[256], "f32", {"gen": ["constf", "-inf"]}],
    [[1024, 1024], "bf16", {"gen": ["triu_fill", 1, "-inf"]}],
    [[3], "i64", {"gen": ["perm"]}],
    ["S", [8, 1024, 512]],
    ["sc", 0.5],
    ["sym", 128],
]


@pytest.mark.parametrize("entry", ENTRIES, ids=[str(e)[:40] for e in ENTRIES])
def test_compact_round_trip(entry):
    assert compact_from_spec(spec_from_compact(entry)) == entry


def test_spec_defaults():
    s = spec_from_compact([[2, 3], "f32"])
    assert s["device"] == "cuda" and s["stride"] == [3, 1] and s["storage_offset"] == 0
    assert "gen" not in s


def test_render_signature():
    sig = render_signature([[[4, 8], "bf16"], ["S", [2, 16]]])
    assert sig.startswith("(T([4, 8], bf16), S([2, 16])")
    from oracle_harness import parse_shapes_signature
    assert parse_shapes_signature(sig) == ((4, 8),)


def test_float_generators_on_cpu():
    torch.manual_seed(0)
    cfg = {"inputs": [spec_from_compact(e) for e in (
        [[20000], "f32", {"gen": ["normal", 0.5, 2.0], "dev": "cpu"}],
        [[64], "f32", {"gen": ["constf", 1.0], "dev": "cpu"}],
        [[5, 7], "bf16", {"gen": ["triu_fill", 1, "-inf"], "dev": "cpu"}],
    )]}
    x, c, m = make_inputs_from_config(cfg)
    assert abs(x.mean().item() - 0.5) < 0.05 and abs(x.std().item() - 2.0) < 0.05
    assert torch.equal(c, torch.ones(64))
    rows, cols = torch.arange(5).view(5, 1), torch.arange(7).view(1, 7)
    assert m.dtype == torch.bfloat16
    assert (m.float()[cols > rows] == -math.inf).all() and (m.float()[cols <= rows] == 0).all()


def test_generation_is_seeded_and_device_independent():
    cfg = {"inputs": [spec_from_compact([[33, 17], "bf16"])]}
    torch.manual_seed(1)
    a = make_inputs_from_config(cfg, device="cpu")[0]
    torch.manual_seed(1)
    b = make_inputs_from_config(cfg, device="cpu")[0]
    assert torch.equal(a, b)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError):
            make_inputs_from_config(cfg)  # spec device is the GPU


def test_strided_and_shape_params():
    cfg = {"inputs": [spec_from_compact([[2, 3, 4, 5], "f32", {"st": [60, 1, 15, 3], "dev": "cpu"}]),
                      spec_from_compact(["S", [6, 20]]), spec_from_compact(["sc", 2.5])]}
    x, s, sc = make_inputs_from_config(cfg)
    assert x.stride() == (60, 1, 15, 3) and s == [6, 20] and sc == 2.5


def test_shape_hash_stable_and_sensitive():
    a = [[[8, 4], "f32"], [[4], "f32"]]
    assert shape_hash_of(a) == shape_hash_of([list(e) for e in a])
    assert shape_hash_of(a) != shape_hash_of([[[8, 4], "bf16"], [[4], "f32"]])
    assert len(shape_hash_of(a)) == 8


def test_instantiate_point():
    point = {"inputs": [[["s0", 64], "f32"], ["S", ["s0 * 2"]]], "bindings": {"s0": 3}}
    symbols = {"s0": {"hint": 4, "range": [1, 10]}}
    assert instantiate_point(point, symbols) == [[[3, 64], "f32"], ["S", [6]]]
    assert instantiate_point(point, symbols, bindings={"s0": 5})[0][0] == [5, 64]
    with pytest.raises(ValueError):
        instantiate_point(point, symbols, bindings={"s0": 11})
    with pytest.raises(ValueError):
        instantiate_point(point, symbols, guards=["s0 > 5"])


def test_shape_hash_is_the_capture_time_identity():
    """Contiguous strides count as "no stride" (torch's rule: size-1 dims
    are free), layouts differ, shape parameters are not part of it."""
    plain = [[[4, 1, 8], "bf16"], [[8], "f32"]]
    assert shape_hash_of(plain) == shape_hash_of([[[4, 1, 8], "bf16", {"st": [8, 8, 1]}], [[8], "f32"]])
    assert shape_hash_of(plain) == shape_hash_of([[[4, 1, 8], "bf16", {"st": [8, 99, 1]}], [[8], "f32"]])
    assert shape_hash_of(plain) == shape_hash_of(plain + [["S", [4, 8]]])
    cl = [[[2, 3, 4, 5], "bf16", {"st": [60, 1, 15, 3]}]]
    assert shape_hash_of(cl) != shape_hash_of([[[2, 3, 4, 5], "bf16"]])
    assert shape_hash_of(plain) == shape_hash_of(list(reversed(plain)))  # sorted descriptors


def test_every_canonical_dir_has_consistent_shapes_json():
    """Every point's hash recomputes from its inputs -- for the corpus
    families this checks the transcription against the reference's own
    capture-time hashes."""
    from conftest import CANONICAL, REPRO_IDS, VARIANT_IDS
    for rid in REPRO_IDS + VARIANT_IDS:
        data = json.loads((CANONICAL / rid / "shapes.json").read_text())
        for p in data["points"]:
            assert p["shape_hash"] == shape_hash_of(p["inputs"]), (rid, p["shape_hash"])
        cfgs = load_shape_configs(str(CANONICAL / rid / "repro.py"))
        assert list(cfgs) == [point_label(p) for p in data["points"]]
        meta = json.loads((CANONICAL / rid / "meta.json").read_text())
        assert meta["origin_ops"]
        if rid in REPRO_IDS:
            assert next(iter(cfgs)).startswith("config"), "BASELINE point first"
            assert meta["pattern_hash"] == rid
        else:
            assert rid.endswith("_" + meta["pattern_hash"])
