"""Pinning the CPU oracle (oracle/hipo_ref.c) -- it is only trusted because
these checks hold.  Each oracle function is checked against:

  * golden fixtures: outputs of PyTorch's eager ATen CPU kernels (the
    arithmetic dependency of the reference's repros, torch 2.10.0 here) on
    tiny seeded inputs, written by tests/golden/make_golden.py;
  * brute force: independent pure-Python evaluations (math module, fp64);
  * closed forms and invariants fixed by the mathematics.

A check that a retyped formula would pass pins nothing, so every check is
also run against deliberately wrong oracles ("planted mistakes": a dropped
term, an off-by-one, a transposed operand) and must reject each of them.
"""
import json
import math
from pathlib import Path

import pytest
import torch

import oracle as ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "aten_eager_small.json").read_text())["cases"]
BF = torch.bfloat16


def from_bits(bits, shape):
    t = torch.tensor(bits, dtype=torch.int32).to(torch.int16).view(BF)
    return t.reshape(shape)


def f32(vals, shape):
    return torch.tensor(vals, dtype=torch.float32).reshape(shape)


def close(a, b, tol):
    a, b = a.float(), b.float()
    return a.shape == b.shape and torch.allclose(a, b, rtol=tol, atol=tol, equal_nan=True)


def bf16_round(v: float) -> float:
    return torch.tensor([v], dtype=torch.float64).to(BF).float().item()


# ---------------------------------------------------------------------------
# Check suites: each takes the function under test and asserts.
# ---------------------------------------------------------------------------

def check_row_mean(fn):
    c = GOLDEN["row_mean"]
    x = f32(c["x"], c["shape"])
    assert close(fn(x), f32(c["out"], [c["shape"][0]]), 1e-6), "golden"
    x = torch.randn(7, 53, generator=torch.Generator().manual_seed(1))
    want = torch.tensor([math.fsum(r) / 53 for r in x.double().tolist()])
    assert close(fn(x), want, 1e-6), "brute force"
    assert torch.equal(fn(torch.full((3, 100), 2.5)), torch.full((3,), 2.5)), "constant rows"
    ar = torch.arange(11, dtype=torch.float32).repeat(2, 1)
    assert torch.equal(fn(ar), torch.full((2,), 5.0)), "mean of 0..10"


def check_bias_gelu(fn):
    c = GOLDEN["bias_gelu_nhwc"]
    n, ch, h, w = c["shape"]
    x, b = from_bits(c["x"], c["shape"]), from_bits(c["bias"], [ch])
    got = fn(x, b)
    assert got.is_contiguous(memory_format=torch.channels_last), "layout"
    want = from_bits(c["out_nhwc"], [n, h, w, ch]).permute(0, 3, 1, 2)
    assert close(got, want, 1.6e-2), "golden"
    exact = (got.float() == want.float()).float().mean().item()
    assert exact > 0.97, f"golden exact fraction {exact}"
    # brute force: t = bf16(x + b); y = 0.5 t (1 + tanh(sqrt(2/pi)(t + 0.044715 t^3)))
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 3, 2, 4, generator=g).to(BF)
    b = torch.randn(3, generator=g).to(BF)
    got = fn(x, b)
    k = math.sqrt(2 / math.pi)
    for i in range(2):
        for c_ in range(3):
            for p in range(8):
                t = bf16_round(x[i, c_].flatten()[p].item() + b[c_].item())
                y = 0.5 * t * (1 + math.tanh(k * (t + 0.044715 * t ** 3)))
                assert abs(got[i, c_].flatten()[p].item() - bf16_round(y)) <= 1e-2 * abs(y) + 1e-6, \
                    "brute force"
    z = torch.zeros(1, 8, 2, 2, dtype=BF)
    assert torch.equal(fn(z, torch.zeros(8, dtype=BF)), z), "gelu(0) = 0"
    big = torch.full((1, 8, 1, 1), 40.0, dtype=BF)
    assert torch.equal(fn(big, torch.zeros(8, dtype=BF)), big), "gelu(t) = t for large t"
    assert (fn(-big, torch.zeros(8, dtype=BF)).float() == 0).all(), "gelu(-large) = 0"


def check_masked_softmax(fn):
    c = GOLDEN["masked_softmax"]
    x, m = from_bits(c["x"], c["shape"]), from_bits(c["mask"], c["shape"][1:])
    want = from_bits(c["out"], c["shape"])
    got = fn(x, m, c["scale"])
    assert close(got, want, 1.6e-2), "golden"
    # brute force on one row: fp64 softmax of bf16-rounded scaled + masked scores
    row = 4
    q = row % c["shape"][1]
    s = [bf16_round(bf16_round(v * c["scale"]) + mv)
         for v, mv in zip(x[0, row].float().tolist(), m[q].float().tolist())]
    mx = max(s)
    e = [math.exp(v - mx) for v in s]
    tot = math.fsum(e)
    assert close(got[0, row], torch.tensor([bf16_round(v / tot) for v in e]), 1e-2), "brute force"
    # uniform scores under a causal mask: 1/(q+1) on j <= q, exactly 0 above
    qn = 9
    causal = torch.triu(torch.full((qn, qn), float("-inf")), 1).to(BF)
    out = fn(torch.full((2, qn, qn), 0.5, dtype=BF), causal, 0.125).float()
    for qi in range(qn):
        assert torch.allclose(out[:, qi, :qi + 1], torch.full((2, qi + 1), bf16_round(1 / (qi + 1))))
        assert (out[:, qi, qi + 1:] == 0).all(), "masked entries are exactly 0"
    sums = fn(torch.randn(3, 8, 40).to(BF), torch.zeros(8, 40, dtype=BF), 0.3).float().sum(-1)
    assert torch.allclose(sums, torch.ones(3, 8), atol=2e-2), "rows sum to 1"


def check_residual_layernorm(fn):
    c = GOLDEN["residual_layernorm"]
    rows, cols = c["shape"]
    args = [from_bits(c[k], [rows, cols]) for k in ("x", "residual")]
    args += [from_bits(c[k], [cols]) for k in ("gamma", "beta")]
    h, y, mean, rstd = fn(*args, c["eps"])
    assert torch.equal(h.view(torch.int16), from_bits(c["h"], [rows, cols]).view(torch.int16)), "h"
    assert close(y, from_bits(c["y"], [rows, cols]), 1.6e-2), "golden y"
    assert close(mean, f32(c["mean"], [rows]), 1e-5), "golden mean"
    assert close(rstd, f32(c["rstd"], [rows]), 1e-5), "golden rstd"
    # brute force on row 2
    hr = h[2].float().tolist()
    mu = math.fsum(hr) / cols
    var = math.fsum((v - mu) ** 2 for v in hr) / cols
    rs = 1 / math.sqrt(var + c["eps"])
    assert abs(mean[2].item() - mu) < 1e-6 and abs(rstd[2].item() - rs) < 1e-5 * rs, "brute force"
    # constant rows: mean = c, var = 0, rstd = 1/sqrt(eps), y = beta
    g_, b_ = torch.randn(16).to(BF), torch.randn(16).to(BF)
    h, y, mean, rstd = fn(torch.full((2, 16), 1.25, dtype=BF), torch.full((2, 16), 0.5, dtype=BF),
                          g_, b_, 1e-5)
    assert torch.equal(mean, torch.full((2,), 1.75))
    assert abs(rstd[0].item() - 1 / math.sqrt(1e-5)) < 1e-2
    assert torch.equal(y, b_.expand(2, 16)), "y = beta"


def check_rmsnorm(fn):
    c = GOLDEN["rmsnorm"]
    rows, cols = c["shape"]
    y, rstd = fn(from_bits(c["x"], [rows, cols]), from_bits(c["gamma"], [cols]), c["eps"])
    assert close(y, from_bits(c["y"], [rows, cols]), 1.6e-2), "golden y"
    assert close(rstd, f32(c["rstd"], [rows]), 1e-5), "golden rstd"
    x = torch.full((1, 8), -3.0, dtype=BF)
    g_ = torch.full((8,), 2.0, dtype=BF)
    y, rs = fn(x, g_, 1e-5)
    assert abs(rs.item() - 1 / math.sqrt(9 + 1e-5)) < 1e-7
    assert torch.allclose(y.float(), torch.full((1, 8), -2.0), atol=1e-2), "y = gamma * sign(x)"


def check_batchnorm(fn):
    c = GOLDEN["batchnorm_train"]
    n, ch, h, w = c["shape"]
    x = f32(c["x"], c["shape"])
    y, sm, si, rm, rv = fn(x, f32(c["gamma"], [ch]), f32(c["beta"], [ch]), torch.zeros(ch),
                           torch.ones(ch), momentum=c["momentum"], eps=c["eps"], relu=True)
    assert close(y, f32(c["y_relu"], c["shape"]), 1e-5), "golden y"
    for k, v in (("save_mean", sm), ("save_invstd", si), ("running_mean", rm), ("running_var", rv)):
        assert close(v, f32(c[k], [ch]), 1e-5), f"golden {k}"
    # two values per channel: x = {0, 2} -> mean 1, biased var 1, unbiased var 2
    x = torch.tensor([0.0, 2.0]).view(2, 1, 1, 1)
    y, sm, si, rm, rv = fn(x, torch.ones(1), torch.zeros(1), torch.zeros(1), torch.ones(1),
                           momentum=0.1, eps=0.0, relu=False)
    assert sm.item() == 1.0 and si.item() == 1.0
    assert torch.equal(y.flatten(), torch.tensor([-1.0, 1.0]))
    assert abs(rm.item() - 0.1) < 1e-7 and abs(rv.item() - (0.9 + 0.1 * 2.0)) < 1e-6, "unbiased"
    # constant channel: var 0 -> y = relu(beta), rm = 0.1 c, rv = 0.9
    x = torch.full((4, 2, 3, 3), 5.0)
    y, sm, si, rm, rv = fn(x, torch.ones(2), torch.tensor([-0.5, 0.5]), torch.zeros(2),
                           torch.ones(2), momentum=0.1, eps=1e-5, relu=True)
    assert torch.equal(y[:, 0], torch.zeros(4, 3, 3)) and torch.allclose(y[:, 1], torch.full((4, 3, 3), 0.5))
    assert torch.allclose(rm, torch.full((2,), 0.5)) and torch.allclose(rv, torch.full((2,), 0.9))


CHECKS = {
    "row_mean": (check_row_mean, ref.row_mean),
    "bias_gelu": (check_bias_gelu, ref.bias_gelu_nchw_to_nhwc),
    "masked_softmax": (check_masked_softmax, ref.scaled_masked_softmax),
    "residual_layernorm": (check_residual_layernorm, ref.residual_layernorm),
    "rmsnorm": (check_rmsnorm, ref.rmsnorm),
    "batchnorm": (check_batchnorm, ref.batchnorm_train),
}


@pytest.mark.parametrize("name", list(CHECKS))
def test_oracle_is_pinned(name):
    check, fn = CHECKS[name]
    check(fn)


# ---------------------------------------------------------------------------
# Planted mistakes: each must be rejected by its check suite.
# ---------------------------------------------------------------------------

def _mean_wrong_divisor(x):
    return ref.row_mean(x) * x.shape[1] / (x.shape[1] - 1)


def _gelu_drops_bias(x, b):
    return ref.bias_gelu_nchw_to_nhwc(x, torch.zeros_like(b))


def _gelu_wrong_layout(x, b):
    return ref.bias_gelu_nchw_to_nhwc(x, b).contiguous()


def _gelu_transposed_bias(x, b):
    return ref.bias_gelu_nchw_to_nhwc(x, b.flip(0))


def _softmax_ignores_mask(x, m, s):
    return ref.scaled_masked_softmax(x, torch.zeros_like(m), s)


def _softmax_ignores_scale(x, m, s):
    return ref.scaled_masked_softmax(x, m, 1.0)


def _ln_no_residual(x, r, g, b, eps):
    return ref.residual_layernorm(x, torch.zeros_like(r), g, b, eps)


def _ln_swapped_affine(x, r, g, b, eps):
    return ref.residual_layernorm(x, r, b, g, eps)


def _rms_ignores_gamma(x, g, eps):
    return ref.rmsnorm(x, torch.ones_like(g), eps)


def _bn_biased_running_var(x, g, b, rm, rv, *, momentum, eps, relu=True):
    y, sm, si, rm2, rv2 = ref.batchnorm_train(x, g, b, rm, rv, momentum=momentum, eps=eps, relu=relu)
    count = x.numel() / x.shape[1]
    rv_biased = (rv2 - (1 - momentum) * rv.float()) * (count - 1) / count + (1 - momentum) * rv.float()
    return y, sm, si, rm2, rv_biased


def _bn_no_relu(x, g, b, rm, rv, *, momentum, eps, relu=True):
    return ref.batchnorm_train(x, g, b, rm, rv, momentum=momentum, eps=eps, relu=False)


MUTANTS = [
    ("row_mean", _mean_wrong_divisor),
    ("bias_gelu", _gelu_drops_bias),
    ("bias_gelu", _gelu_wrong_layout),
    ("bias_gelu", _gelu_transposed_bias),
    ("masked_softmax", _softmax_ignores_mask),
    ("masked_softmax", _softmax_ignores_scale),
    ("residual_layernorm", _ln_no_residual),
    ("residual_layernorm", _ln_swapped_affine),
    ("rmsnorm", _rms_ignores_gamma),
    ("batchnorm", _bn_biased_running_var),
    ("batchnorm", _bn_no_relu),
]


@pytest.mark.parametrize("name,mutant", MUTANTS, ids=[m.__name__ for _, m in MUTANTS])
def test_planted_mistake_is_caught(name, mutant):
    check, _ = CHECKS[name]
    with pytest.raises(AssertionError):
        check(mutant)


def test_oracle_matches_repro_eager_modules():
    """The oracle agrees with the build's own repro modules (eager ATen) on
    their ragged shapes.json points, generated on the CPU."""
    from conftest import CANONICAL, REPRO_IDS
    from oracle_harness import _normalize_outputs, get_repro_instance
    from repro_harness import load_shape_configs, make_inputs_from_config
    calls = {
        "mean_lastdim_f32": lambda i: [ref.row_mean(i[0])],
        "pointwise_bias_gelu_tanh_nhwc": lambda i: [ref.bias_gelu_nchw_to_nhwc(*i)],
        "amax_sum_scaled_masked_softmax": lambda i: [ref.scaled_masked_softmax(i[0], i[1], 0.125)],
        "var_mean_residual_layernorm": lambda i: list(ref.residual_layernorm(*i, 1e-5)),
        "mean_rmsnorm": lambda i: list(ref.rmsnorm(*i, 1e-5)),
        "var_mean_batchnorm_train_relu": lambda i: list(
            ref.batchnorm_train(*i, momentum=0.1, eps=1e-5)),
    }
    for rid in REPRO_IDS:
        inst = get_repro_instance(CANONICAL / rid)
        for label, cfg in list(load_shape_configs(str(CANONICAL / rid / "repro.py")).items())[1:]:
            torch.manual_seed(1)
            inp = make_inputs_from_config(cfg, device="cpu")
            want = _normalize_outputs(inst(*[t.clone() for t in inp]))
            got = calls[rid](inp)
            for i, (g, w) in enumerate(zip(got, want)):
                tol = 1.6e-2 if w.dtype == BF else 1e-5
                assert close(g, w, tol), f"{rid}/{label} out{i}"
