"""oracle_impl / OracleRegistry dispatch, restating the assertions of the
reference's tests/test_oracle_dispatch.py:66-219 (signature parsing, every
match level, exact-only matching, configs passthrough, dtype honesty, empty
signatures, unmigrated modules) plus the MI355X hardware kind and hash-keyed
registrations against this build's shapes.json files."""
import pytest
import torch

import oracle_harness
from oracle_harness import (OracleDispatchError, oracle_impl, parse_shapes_signature,
                            reset_oracle_registry, resolve_oracle)

MOD = "test_oracle_dispatch_fake"
CALLS = []


def fake_inputs(*shapes, dtype=torch.float32):
    return [torch.empty(s, dtype=dtype, device="meta") for s in shapes]


def make(name, expect_configs=False):
    if expect_configs:
        def fn(inputs, **cfg):
            CALLS.append((name, cfg))
            return name
    else:
        def fn(inputs):
            CALLS.append((name, None))
            return name
    fn.__module__ = MOD
    fn.__name__ = name
    return fn


@pytest.fixture(autouse=True)
def fresh(monkeypatch):
    monkeypatch.setattr(oracle_harness.get_gpu_kind, "_cached", "MI355X", raising=False)
    reset_oracle_registry(MOD)
    CALLS.clear()
    yield
    reset_oracle_registry(MOD)


def test_parse_shapes_signature():
    sig = parse_shapes_signature(
        "(T([512, 256, 13, 13], f32), T([512, 128, 27, 27], b8), S([131072, 169]))")
    assert sig == ((512, 256, 13, 13), (512, 128, 27, 27))
    assert parse_shapes_signature(None) is None
    assert parse_shapes_signature(((8, 4), (4,))) == ((8, 4), (4,))
    assert parse_shapes_signature("(T([8192, 262144], bf16))") == ((8192, 262144),)
    assert parse_shapes_signature("(T([8, 512], i64, gen=Index(32128)),)") == ((8, 512),)
    shapes, dtypes = parse_shapes_signature("(T([4], bf16), T([2, 2], f32))", with_dtypes=True)
    assert shapes == ((4,), (2, 2)) and dtypes == ("bf16", "f32")


def test_hardware_and_shape_match():
    oracle_impl(hardware="MI355X", shapes="(T([32768, 1024], bf16),)")(make("mi355x"))
    oracle_impl(hardware="B200", shapes="(T([32768, 1024], bf16),)")(make("b200"))
    _, info = resolve_oracle(make("entry"), fake_inputs((32768, 1024)))
    assert info["matched"] == "hardware+shape" and info["fn_name"] == "mi355x"
    assert not info["fallback"] and info["current_hardware"] == "MI355X"


def test_shape_match_other_hardware_is_fallback():
    oracle_impl(hardware="B200", shapes="(T([32768, 1024], bf16),)")(make("b200"))
    _, info = resolve_oracle(make("entry"), fake_inputs((32768, 1024)))
    assert info["matched"] == "shape" and info["fallback"] and info["tuned_hardware"] == "B200"
    _, info = resolve_oracle(make("entry"), fake_inputs((32768, 1024), dtype=torch.float16))
    assert info["matched"] == "shape"  # dtype is not a match requirement


def test_wrong_shape_raises():
    oracle_impl(hardware="MI355X", shapes="(T([32768, 1024], bf16),)")(make("strict"))
    with pytest.raises(OracleDispatchError):
        resolve_oracle(make("entry"), fake_inputs((32768, 4096)))


def test_shape_general_levels():
    oracle_impl(hardware="MI355X")(make("general_mi355x"))
    _, info = resolve_oracle(make("entry"), fake_inputs((7, 9)))
    assert info["matched"] == "hardware" and info["fallback"]
    reset_oracle_registry(MOD)
    oracle_impl(hardware="B200", shapes="(T([4], f32),)")(make("strict"))
    oracle_impl()(make("default"))
    _, info = resolve_oracle(make("entry"), fake_inputs((7, 7)))
    assert info["matched"] == "any" and info["fn_name"] == "default"


def test_exact_shape_beats_shape_general():
    oracle_impl(hardware="MI355X")(make("general"))
    oracle_impl(hardware="B200", shapes="(T([32768, 1024], bf16),)")(make("tuned_b200"))
    _, info = resolve_oracle(make("entry"), fake_inputs((32768, 1024)))
    assert info["fn_name"] == "tuned_b200" and info["matched"] == "shape"


def test_configs_passthrough_per_shape_and_hardware():
    shared = make("shared", expect_configs=True)
    oracle_impl(hardware="MI355X", shapes="(T([32768, 256], bf16),)", BLOCK=256)(shared)
    oracle_impl(hardware="MI355X", shapes="(T([8192, 262144], bf16),)", BLOCK=4096)(shared)
    oracle_impl(hardware="B200", shapes="(T([8192, 262144], bf16),)", BLOCK=1)(shared)
    fn, info = resolve_oracle(make("entry"), fake_inputs((8192, 262144)))
    assert info["matched"] == "hardware+shape"
    fn(fake_inputs((8192, 262144)))
    assert CALLS[-1] == ("shared", {"BLOCK": 4096})
    fn, _ = resolve_oracle(make("entry"), fake_inputs((32768, 256)))
    fn(fake_inputs((32768, 256)))
    assert CALLS[-1] == ("shared", {"BLOCK": 256})


def test_multi_tensor_signature_and_count_mismatch():
    oracle_impl(hardware="MI355X", shapes="(T([1024, 64], f32), T([64], f32))")(make("two"))
    _, info = resolve_oracle(make("entry"), fake_inputs((1024, 64), (64,)))
    assert info["matched"] == "hardware+shape"
    with pytest.raises(OracleDispatchError):
        resolve_oracle(make("entry"), fake_inputs((1024, 64)))


def test_dtype_honesty_flag():
    oracle_impl(hardware="MI355X", shapes="(T([32768, 1024], bf16),)")(make("bf16_tuned"))
    _, info = resolve_oracle(make("entry"), fake_inputs((32768, 1024), dtype=torch.float32))
    assert info.get("dtypes_differ") is True
    assert info["tuned_dtypes"] == ("bf16",) and info["actual_dtypes"] == ("f32",)
    _, info = resolve_oracle(make("entry"), fake_inputs((32768, 1024), dtype=torch.bfloat16))
    assert "dtypes_differ" not in info


def test_empty_and_shape_param_only_signatures():
    oracle_impl(hardware="B200", shapes="()")(make("no_tensors"))
    _, info = resolve_oracle(make("entry"), [512, 3.0])
    assert info["matched"] == "shape" and info["fn_name"] == "no_tensors"
    reset_oracle_registry(MOD)
    oracle_impl(hardware="B200", shapes="(S([1, -1, 512, 512]))")(make("s_only"))
    _, info = resolve_oracle(make("entry"), [512])
    assert info["fn_name"] == "s_only"


def test_unmigrated_module_untouched():
    def plain(inputs):
        return "plain"
    plain.__module__ = "some_unmigrated_module"
    fn, info = resolve_oracle(plain, fake_inputs((3, 3)))
    assert fn is plain and info is None


def test_callable_shape_and_bad_configs_rejected():
    reg = oracle_harness.OracleRegistry()
    with pytest.raises(TypeError):
        reg.register(shape=lambda s: True)
    with pytest.raises(TypeError):
        reg.register(configs=[1, 2])
    with pytest.raises(ValueError):
        oracle_impl(point="abcd1234", shapes="(T([4], f32),)")


def test_gpu_kind_from_device_name(monkeypatch):
    class Props:
        def __init__(self, name, arch):
            self.name, self.gcnArchName = name, arch
    monkeypatch.delattr(oracle_harness.get_gpu_kind, "_cached", raising=False)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i: Props("AMD Instinct MI355X", "gfx950:sramecc+:xnack-"))
    assert oracle_harness.get_gpu_kind() == "MI355X"
    monkeypatch.delattr(oracle_harness.get_gpu_kind, "_cached")
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i: Props("", "gfx950"))
    assert oracle_harness.get_gpu_kind() == "MI355X"
    monkeypatch.delattr(oracle_harness.get_gpu_kind, "_cached")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert oracle_harness.get_gpu_kind() == "unknown"


def test_build_oracles_register_their_points():
    """Every gfx950 oracle.py registers its BASELINE point (by shape_hash of
    the sibling shapes.json) and a shape-general MI355X variant."""
    import json
    from conftest import CANONICAL, REPRO_IDS
    for rid in REPRO_IDS:
        mod, fn, d = oracle_harness._load_oracle_module(CANONICAL / rid)
        reg = oracle_harness.get_module_registry(mod.__name__)
        entries = reg.list_entries()
        assert len(entries) == 2, entries
        assert {e["hardware"] for e in entries} == {"MI355X"}
        points = json.loads((d / "shapes.json").read_text())["points"]
        specs = [s for s in points[0]["inputs"]]
        baseline_shapes = tuple(tuple(s[0]) for s in specs)
        assert any(e["shape"] == baseline_shapes for e in entries)
        meta = [torch.empty(s, device="meta") for s in baseline_shapes]
        _, info = resolve_oracle(fn, meta)
        assert info["matched"] == "hardware+shape"
        # re-loading the module does not register twice
        mod, fn, d = oracle_harness._load_oracle_module(CANONICAL / rid)
        assert len(oracle_harness.get_module_registry(mod.__name__).list_entries()) == 2
