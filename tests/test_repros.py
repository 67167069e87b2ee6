"""The build's repro modules restate the BASELINE configs with eager ATen
semantics: check them against the ATen functions they decompose, and that
every repro follows the canonical-repro contract (Repro, make_inputs,
shapes.json default point).  CPU only, small ragged points."""
import pytest
import torch
import torch.nn.functional as F

from conftest import CANONICAL, REPRO_IDS
from oracle_harness import get_repro_instance, load_repro_module
from repro_harness import load_shape_configs, make_inputs_from_config


def small_inputs(rid, idx=1):
    cfg = list(load_shape_configs(str(CANONICAL / rid / "repro.py")).values())[idx]
    torch.manual_seed(3)
    return make_inputs_from_config(cfg, device="cpu")


def test_rmsnorm_repro_equals_functional_rms_norm():
    x, g = small_inputs("mean_rmsnorm")
    y, rstd = get_repro_instance(CANONICAL / "mean_rmsnorm")(x, g)
    assert torch.equal(y, F.rms_norm(x, [x.shape[-1]], g, 1e-5))
    assert torch.allclose(rstd, torch.rsqrt(x.float().pow(2).mean(-1) + 1e-5))


def test_layernorm_repro_matches_functional_layer_norm():
    x, r, g, b = small_inputs("var_mean_residual_layernorm")
    h, y, mean, rstd = get_repro_instance(CANONICAL / "var_mean_residual_layernorm")(x, r, g, b)
    assert torch.equal(h, x + r)
    want = F.layer_norm(h.float(), [h.shape[-1]], g.float(), b.float(), 1e-5).to(torch.bfloat16)
    assert (y.float() - want.float()).abs().max() <= 1.6e-2 * want.float().abs().max()
    assert torch.allclose(mean, h.float().mean(-1), atol=1e-6)


def test_gelu_repro_is_channels_last_tanh_gelu():
    x, b = small_inputs("pointwise_bias_gelu_tanh_nhwc")
    y = get_repro_instance(CANONICAL / "pointwise_bias_gelu_tanh_nhwc")(x, b)
    assert y.is_contiguous(memory_format=torch.channels_last)
    assert torch.equal(y, F.gelu(x + b.view(1, -1, 1, 1), approximate="tanh"))


def test_softmax_repro():
    x, m = small_inputs("amax_sum_scaled_masked_softmax")
    y = get_repro_instance(CANONICAL / "amax_sum_scaled_masked_softmax")(x, m)
    assert torch.equal(y, torch.softmax(x * 0.125 + m, -1))


def test_batchnorm_repro_updates_running_stats_in_place():
    x, g, b, rm, rv = small_inputs("var_mean_batchnorm_train_relu")
    rm0, rv0 = rm.clone(), rv.clone()
    y, sm, si, rm_out, rv_out = get_repro_instance(CANONICAL / "var_mean_batchnorm_train_relu")(
        x, g, b, rm, rv)
    assert rm_out is rm and rv_out is rv and not torch.equal(rm, rm0)
    ref = F.batch_norm(x, rm0, rv0, g, b, training=True, momentum=0.1, eps=1e-5)
    assert torch.allclose(y, torch.relu(ref), atol=1e-5)
    assert torch.allclose(rm, rm0) and torch.allclose(rv, rv0)  # F.batch_norm updated the copies


def test_fp64_copy_computes_in_fp64():
    """Repro().double() on fp64 inputs must not round back to fp32/bf16
    (the numerics gate's reference)."""
    for rid in ("var_mean_residual_layernorm", "mean_rmsnorm"):
        inp = [t.double() for t in small_inputs(rid)]
        outs = get_repro_instance(CANONICAL / rid).double()(*inp)
        assert all(o.dtype == torch.float64 for o in outs), rid


@pytest.mark.parametrize("rid", REPRO_IDS)
def test_repro_contract(rid):
    mod = load_repro_module(CANONICAL / rid)
    assert hasattr(mod, "Repro") and hasattr(mod, "make_inputs") and mod._repro_version == 3
    cfgs = load_shape_configs(str(CANONICAL / rid / "repro.py"))
    assert len(cfgs) >= 3
    small = list(cfgs.values())[2]
    torch.manual_seed(0)
    out = mod.Repro()(*make_inputs_from_config(small, device="cpu"))
    assert out is not None
