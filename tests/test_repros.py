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


# ---------------------------------------------------------------------------
# Corpus families (the reference's canonical dirs; small inputs of the same
# structure, checked against independent formulations)
# ---------------------------------------------------------------------------

from conftest import LN_FAMILY_OUTPUTS, RMS_FAMILY_OUTPUTS, VARIANT_IDS  # noqa: E402

bf = torch.bfloat16


def test_spatial_mean_family_repro():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 40, 5, 6, generator=g).to(bf).contiguous(memory_format=torch.channels_last)
    y = get_repro_instance(CANONICAL / "mean_c9e1a8113328")(x)
    assert y.shape == (3, 40, 1, 1) and y.dtype == bf
    assert torch.equal(y, x.mean(dim=(2, 3), keepdim=True))


def test_t5_rmsnorm_family_repro():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(6, 64, generator=g).to(bf)
    r = torch.randn(2, 3, 64, generator=g).to(bf)
    w = torch.randn(64, generator=g).to(bf)
    y = get_repro_instance(CANONICAL / "mean_4462ce967d63")(x, r, w, [2, 3, 64], [6, 64])
    h = (r + x.view(2, 3, 64)).float()
    rstd = torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)
    normed = (h * rstd).to(bf)
    want = ((w * normed) * 0.04419417382415922).view(6, 64)
    assert torch.equal(y, want) and y.dtype == bf


def test_bias_softmax_family_repro():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(8, 5, 12, generator=g).to(bf)      # 2 groups x 4 heads
    b = torch.randn(2, 1, 5, 12, generator=g).to(bf)
    y = get_repro_instance(CANONICAL / "amax_sum_20ccc18dda60")(x, b, [2, 4, 5, 12], [8, 5, 12])
    want = torch.softmax((x.view(2, 4, 5, 12) + b).float(), -1).to(bf).view(8, 5, 12)
    assert torch.equal(y, want)


def test_plain_softmax_family_repro():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(6, 5, 12, generator=g).to(bf)      # viewed [2, 3, 5, 12]
    y = get_repro_instance(CANONICAL / "amax_sum_fa4cc85fe5ad")(
        x, [2, 3, 5, 12], [2, 3, 5, 12], [6, 5, 12])
    assert y.shape == (6, 5, 12) and y.dtype == bf
    assert torch.equal(y, torch.softmax(x.float(), -1).to(bf))


def test_gelu_bwd_family_repro():
    """GELU(erf) backward + column sum: y against ATen's own gelu_backward
    (fp32, within a bf16 rounding), its transpose a view of y, the column sum
    the bf16 rounding of y's fp32 column sum."""
    g = torch.Generator().manual_seed(21)
    grad = torch.randn(12, 16, generator=g).to(bf)
    x = (2 * torch.randn(12, 16, generator=g)).to(bf)
    y, yt, colsum = get_repro_instance(CANONICAL / "sum_139a3020e8bf")(
        grad, x, [3, 4, 16], [3, 4, 16], [12, 16], [16])
    want = torch.ops.aten.gelu_backward(grad.float(), x.float())
    assert y.shape == (12, 16) and y.dtype == bf
    assert (y.float() - want).abs().max() <= 2 ** -8 * want.abs().max()
    assert yt.shape == (16, 12) and yt.data_ptr() == y.data_ptr() and torch.equal(yt, y.t())
    assert colsum.dtype == torch.float32 and colsum.shape == (16,)
    assert torch.equal(colsum, y.float().sum(0).to(bf).float())


@pytest.mark.parametrize("rid", sorted(LN_FAMILY_OUTPUTS))
def test_residual_layernorm_family_repros(rid):
    """Each residual-LayerNorm family repro at a small shape of its own
    signature: outputs (count, shape, aliasing) as LN_FAMILY_OUTPUTS says,
    values against F.layer_norm of the bf16 sum in fp32."""
    mod = load_repro_module(CANONICAL / rid)
    kind = LN_FAMILY_OUTPUTS[rid]
    g = torch.Generator().manual_seed(sum(map(ord, rid)))
    b, t, c = 2, 3, 64
    two_d = False  # every family here passes the residual as [b, t, c]
    x = torch.randn(b * t, c, generator=g).to(bf)
    r = (torch.randn(b * t, c, generator=g) if two_d else torch.randn(b, t, c, generator=g)).to(bf)
    w, beta = torch.randn(c, generator=g).to(bf), torch.randn(c, generator=g).to(bf)
    nshape = {"y2": 2, "h_y2": 2, "h_y2x3": 4, "y3_y2x3": 4, "y3_y2": 2}[kind]
    shapes = [[b, t, c]] + [[b * t, c]] * (nshape - 1)
    out = get_repro_instance(CANONICAL / rid)(x, r, w, beta, *shapes)
    out = list(out) if isinstance(out, tuple) else [out]
    h = (x.view(b, t, c) + r.view(b, t, c))
    y = F.layer_norm(h.float(), [c], w.float(), beta.float(), mod.EPS).to(bf)
    close = lambda a, e: (a.float() - e.float()).abs().max() <= 1.6e-2 * e.float().abs().max()
    if kind.startswith("h_"):
        assert torch.equal(out[0], h.view(r.shape)) and out[0].shape == r.shape
        ys = out[1:]
    else:
        ys = out
    assert len(ys) == {"y2": 1, "h_y2": 1, "h_y2x3": 3, "y3_y2x3": 4, "y3_y2": 2}[kind]
    for k, yk in enumerate(ys):
        assert yk.dtype == bf and close(yk.reshape(b, t, c), y)
        if kind.startswith("y3") and k == 0:
            assert yk.shape == (b, t, c)
        else:
            assert yk.shape == (b * t, c)
    assert len({yk.data_ptr() for yk in ys}) == 1, "the y outputs are views of one tensor"


@pytest.mark.parametrize("rid", sorted(RMS_FAMILY_OUTPUTS))
def test_residual_rmsnorm_family_repros(rid):
    """Each residual-RMSNorm family repro at a small shape of its signature:
    outputs as RMS_FAMILY_OUTPUTS says (h exact, the y views of one tensor),
    y against the graph's op order written out in fp32 / bf16."""
    mod = load_repro_module(CANONICAL / rid)
    mode, first, nviews = RMS_FAMILY_OUTPUTS[rid]
    g = torch.Generator().manual_seed(sum(map(ord, rid)))
    b, t, c = 2, 3, 64
    x = torch.randn(b * t, c, generator=g).to(bf)
    r = torch.randn(b, t, c, generator=g).to(bf)
    w = torch.randn(c, generator=g).to(bf)
    shapes = [[b, t, c]] + [[b * t, c]] * nviews
    out = get_repro_instance(CANONICAL / rid)(x, r, w, *shapes)
    out = list(out) if isinstance(out, tuple) else [out]
    h = x.view(b, t, c) + r
    rstd = torch.rsqrt(h.float().pow(2).mean(-1, keepdim=True) + mod.EPS)
    if mode == 1:
        y = w * (h.float() * rstd).to(bf)
    else:
        y = (w.float() * (h.float() * rstd)).to(bf)
    assert len(out) == (1 if first else 0) + nviews
    if first == "h":
        assert torch.equal(out[0], h)
    elif first == "y":
        assert torch.equal(out[0], y)
    views = out[1:] if first else out
    for v in views:
        assert v.shape == (b * t, c) and torch.equal(v, y.view(b * t, c))
    ys = [o for o in out if not (first == "h" and o is out[0])]
    assert len({o.data_ptr() for o in ys}) == 1, "the y outputs are views of one tensor"


def test_longformer_layernorm_family_repro():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(6, 32, generator=g).to(bf)
    r = torch.randn(2, 3, 32, generator=g).to(bf)
    w, b = torch.randn(32, generator=g).to(bf), torch.randn(32, generator=g).to(bf)
    y = get_repro_instance(CANONICAL / "var_mean_80e7ff4dee7f")(x, r, w, b, [2, 3, 32])
    h = (x.view(2, 3, 32) + r).float()
    want = F.layer_norm(h, [32], w.float(), b.float(), 1e-5).to(bf)
    assert y.shape == (2, 3, 32)
    assert (y.float() - want.float()).abs().max() <= 1.6e-2 * want.float().abs().max()


def test_family_repros_compute_in_fp64_for_the_gate():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(6, 64, generator=g).double()
    r = torch.randn(2, 3, 64, generator=g).double()
    w = torch.randn(64, generator=g).double()
    y = get_repro_instance(CANONICAL / "mean_4462ce967d63").double()(x, r, w, [2, 3, 64], [6, 64])
    assert y.dtype == torch.float64
    b = torch.randn(64, generator=g).double()
    y = get_repro_instance(CANONICAL / "var_mean_80e7ff4dee7f").double()(x, r, w, b, [2, 3, 64])
    assert y.dtype == torch.float64


@pytest.mark.parametrize("rid", VARIANT_IDS)
def test_family_repro_contract(rid):
    mod = load_repro_module(CANONICAL / rid)
    assert hasattr(mod, "Repro") and hasattr(mod, "make_inputs") and mod._repro_version == 3
    cfgs = load_shape_configs(str(CANONICAL / rid / "repro.py"))
    assert len(cfgs) >= 1
    import json
    meta = json.loads((CANONICAL / rid / "meta.json").read_text())
    assert rid.endswith(meta["pattern_hash"])
    # every shapes.json point has an MI355X registration -- its own, or, where
    # points differ only in strides (the registry keys by input shapes), that
    # of a point with the same input shapes -- plus one shape-general entry
    # for shapes outside the corpus; except the points the module withdraws
    # (WITHDRAWN_POINTS), which match no entry: such a dir has no
    # shape-general entry either
    import oracle_harness as oh
    mod, fn, _ = oh._load_oracle_module(CANONICAL / rid)
    entries = oh.get_module_registry(fn.__module__)._entries
    points = json.loads((CANONICAL / rid / "shapes.json").read_text())["points"]
    withdrawn = getattr(mod, "WITHDRAWN_POINTS", {})
    hashes = {p["shape_hash"] for p in points}
    assert set(withdrawn) <= hashes

    def shapes(p):
        return tuple(tuple(i[0]) for i in p["inputs"] if i[0] != "S")
    registered = {e["point"] for e in entries if e["point"]}
    assert registered <= hashes and not registered & set(withdrawn)
    covered = {shapes(p) for p in points if p["shape_hash"] in registered}
    assert all(shapes(p) in covered for p in points if p["shape_hash"] not in withdrawn)
    general = any(e["shape"] is None and e["hardware"] == "MI355X" for e in entries)
    assert general == (not withdrawn)
    for label, pcfg in cfgs.items():
        if label.rsplit("_", 1)[-1] in withdrawn:
            with pytest.raises(oh.OracleDispatchError):
                oh.resolve_oracle(fn, make_inputs_from_config(pcfg, device="meta"))


def _bn_inputs(shape, memory_format, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * 2 + 0.5).to(bf).contiguous(memory_format=memory_format)
    c = shape[1]
    rm, rv = torch.randn(c, generator=g), torch.rand(c, generator=g) + 0.5
    gamma, beta = torch.randn(c, generator=g), torch.randn(c, generator=g)
    return x, rm, rv, gamma, beta


def test_bn_silu_pad_family_repro():
    x, rm, rv, gamma, beta = _bn_inputs((3, 16, 5, 6), torch.channels_last, 10)
    rm0, rv0 = rm.clone(), rv.clone()
    mean, rstd, out, rm_out, rv_out = get_repro_instance(CANONICAL / "var_mean_ceb5c315290a")(
        x, rm, rv, gamma, beta)
    assert rm_out is rm and rv_out is rv
    assert out.shape == (3, 16, 6, 7) and out.is_contiguous(memory_format=torch.channels_last)
    y = F.batch_norm(x.float(), None, None, gamma, beta, training=True, eps=1e-3).to(bf)
    assert torch.equal(out, F.pad(F.silu(y.float()).to(bf), (0, 1, 0, 1)))
    var, m = torch.var_mean(x.float(), [0, 2, 3], correction=0)
    assert mean.shape == rstd.shape == (1, 16, 1, 1)
    assert torch.allclose(mean.flatten(), m) and torch.allclose(rstd.flatten(), torch.rsqrt(var + 1e-3))
    # the graph's Bessel constant, not N/(N-1) of this shape
    assert torch.allclose(rm, m * 0.1 + rm0 * 0.9)
    assert torch.allclose(rv, var * 1.00000996502277 * 0.1 + rv0 * 0.9)


def test_bn_relu_mean_family_repro():
    x, rm, rv, gamma, beta = _bn_inputs((5, 12, 7, 7), torch.contiguous_format, 11)
    rm0, rv0 = rm.clone(), rv.clone()
    mean, rstd, out, rm_out, rv_out = get_repro_instance(CANONICAL / "var_mean_mean_19ffdb35cc67")(
        x, rm, rv, gamma, beta)
    assert rm_out is rm and rv_out is rv
    y = F.batch_norm(x.float(), None, None, gamma, beta, training=True, eps=1e-5).to(bf)
    want = torch.relu(y).mean((2, 3))
    assert out.shape == (5, 12) and out.dtype == bf
    assert torch.equal(out, want)
    var, m = torch.var_mean(x.float(), [0, 2, 3], correction=0)
    assert torch.allclose(rm, m * 0.1 + rm0 * 0.9)
    assert torch.allclose(rv, var * 1.0001594642002871 * 0.1 + rv0 * 0.9)


def test_bn_family_repros_compute_in_fp64_for_the_gate():
    for rid, fmt in (("var_mean_ceb5c315290a", torch.channels_last),
                     ("var_mean_mean_19ffdb35cc67", torch.contiguous_format)):
        inp = [t.double() for t in _bn_inputs((2, 8, 4, 4), fmt, 12)]
        outs = get_repro_instance(CANONICAL / rid).double()(*inp)
        assert all(o.dtype == torch.float64 for o in outs), rid
