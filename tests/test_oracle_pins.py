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
    # brute force on one row: fp64 softmax of the unrounded scores x * scale + mask
    row = 4
    q = row % c["shape"][1]
    s = [v * c["scale"] + mv for v, mv in zip(x[0, row].float().tolist(), m[q].float().tolist())]
    mx = max(s)
    e = [math.exp(v - mx) for v in s]
    tot = math.fsum(e)
    want_row = torch.tensor([bf16_round(v / tot) for v in e])
    assert close(got[0, row], want_row, 1e-2), "brute force"
    assert (got[0, row].float() == want_row).float().mean().item() > 0.97, "brute force, exact"
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


def from_nhwc_bits(bits, shape):
    n, c, h, w = shape
    return from_bits(bits, [n, h, w, c]).permute(0, 3, 1, 2)


def exact_fraction(a, b):
    return (a.float() == b.float()).float().mean().item()


def check_spatial_mean(fn):
    c = GOLDEN["spatial_mean_nhwc"]
    x = from_nhwc_bits(c["x_nhwc"], c["shape"])
    got = fn(x)
    want = from_bits(c["out"], [c["shape"][0], c["shape"][1], 1, 1])
    assert close(got, want, 1.6e-2) and exact_fraction(got, want) > 0.9, "golden"
    # brute force: fp64 sum over positions of each (image, channel)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(2, 5, 3, 7, generator=g) * 3).to(BF)
    got = fn(x)
    for i in range(2):
        for ch in range(5):
            v = math.fsum(x[i, ch].float().flatten().tolist()) / 21
            assert abs(got[i, ch, 0, 0].item() - bf16_round(v)) <= 1e-2 * abs(v) + 1e-6, "brute force"
    const = torch.full((3, 16, 4, 4), 0.625, dtype=BF)
    assert torch.equal(fn(const), torch.full((3, 16, 1, 1), 0.625, dtype=BF)), "constant"


def check_bias_softmax(fn):
    c = GOLDEN["bias_softmax"]
    b_, q, k = c["shape"]
    heads = c["heads"]
    x, bias = from_bits(c["x"], c["shape"]), from_bits(c["bias"], [b_ // heads, q, k])
    got = fn(x, bias, c["scale"], heads)
    assert close(got, from_bits(c["out"], c["shape"]), 1.6e-2), "golden"
    # brute force, batch entry 4 (group 1), row 2
    s = [bf16_round(bf16_round(v * c["scale"]) + bv)
         for v, bv in zip(x[4, 2].float().tolist(), bias[4 // heads, 2].float().tolist())]
    mx = max(s)
    e = [math.exp(v - mx) for v in s]
    tot = math.fsum(e)
    assert close(got[4, 2], torch.tensor([bf16_round(v / tot) for v in e]), 1e-2), "brute force"
    # group mapping: bias group j is -inf except column j -> out[b] one-hot at b // heads
    groups, hh = 3, 4
    onehot_bias = torch.full((groups, 2, 8), float("-inf"))
    for j in range(groups):
        onehot_bias[j, :, j] = 0
    out = fn(torch.randn(groups * hh, 2, 8).to(BF), onehot_bias.to(BF), 1.0, hh).float()
    for bb in range(groups * hh):
        want = torch.zeros(2, 8)
        want[:, bb // hh] = 1
        assert torch.equal(out[bb], want), f"batch {bb} uses bias group {bb // hh}"


def check_rmsnorm_ex(fn):
    c = GOLDEN["rmsnorm_t5"]
    rows, cols = c["shape"]
    x, r = from_bits(c["x"], [rows, cols]), from_bits(c["residual"], [rows, cols])
    gm = from_bits(c["gamma"], [cols])
    y, rstd = fn(x, gm, c["eps"], residual=r, scale=c["scale"], mode=1)
    want = from_bits(c["y"], [rows, cols])
    assert close(y, want, 1.6e-2), "golden T5 y"
    assert exact_fraction(y, want) > 0.97, f"golden T5 exact {exact_fraction(y, want)}"
    assert close(rstd, f32(c["rstd"], [rows]), 1e-5), "golden rstd"
    y0, _ = fn(x, gm, c["eps"], residual=r, mode=0)
    want0 = from_bits(c["y_residual_rms_norm"], [rows, cols])
    assert close(y0, want0, 1.6e-2) and exact_fraction(y0, want0) > 0.97, "golden rms_norm(x + r)"
    # brute force row 3, T5 order
    h = [bf16_round(a + b) for a, b in zip(x[3].float().tolist(), r[3].float().tolist())]
    rs = 1 / math.sqrt(math.fsum(v * v for v in h) / cols + c["eps"])
    for j in range(cols):
        u = bf16_round(gm[j].item() * bf16_round(h[j] * rs))
        assert abs(y[3, j].item() - bf16_round(u * c["scale"])) <= 1e-2 * abs(u * c["scale"]) + 1e-6
    # constant rows: rstd = 1/sqrt(c^2 + eps); gamma = 1 -> y = bf16(c * rstd) * scale
    yc, rc = fn(torch.full((2, 16), 3.0, dtype=BF), torch.ones(16, dtype=BF), 1e-6,
                scale=0.5, mode=1)
    assert abs(rc[0].item() - 1 / math.sqrt(9 + 1e-6)) < 1e-7
    assert torch.equal(yc, torch.full((2, 16), 0.5, dtype=BF))


def check_bn_nhwc(fn):
    c = GOLDEN["bn_nhwc_silu_pad"]
    n, ch, h, w = c["shape"]
    x = from_nhwc_bits(c["x_nhwc"], c["shape"])
    sm, sr, out, rm, rv = fn(x, f32(c["gamma"], [ch]), f32(c["beta"], [ch]),
                             f32(c["running_mean"], [ch]), f32(c["running_var"], [ch]),
                             momentum=c["momentum"], eps=c["eps"], var_scale=c["var_scale"],
                             act="silu", pad_bottom=1, pad_right=1)
    want = from_nhwc_bits(c["out_nhwc"], [n, ch, h + 1, w + 1])
    assert out.shape == want.shape and out.is_contiguous(memory_format=torch.channels_last)
    assert close(out, want, 1.6e-2), "golden out"
    for key, v in (("save_mean", sm), ("save_rstd", sr), ("running_mean_out", rm),
                   ("running_var_out", rv)):
        assert close(v.flatten(), f32(c[key], [ch]), 1e-5), f"golden {key}"
    assert (out[:, :, h:, :].float() == 0).all() and (out[:, :, :, w:].float() == 0).all(), "pad"
    # constant channel: var 0 -> y = silu(bf16(beta)); running_var decays
    x = torch.full((2, 4, 3, 3), 1.5, dtype=BF).contiguous(memory_format=torch.channels_last)
    beta = torch.tensor([-1.0, 0.0, 0.5, 2.0])
    sm, sr, out, rm, rv = fn(x, torch.ones(4), beta, torch.zeros(4), torch.ones(4), momentum=0.1,
                             eps=1e-3, var_scale=2.0, act="silu", pad_bottom=1, pad_right=1)
    silu = [bf16_round(v / (1 + math.exp(-v))) for v in beta.tolist()]
    assert torch.allclose(out[:, :, :3, :3].float(), torch.tensor(silu).view(1, 4, 1, 1).expand(2, 4, 3, 3))
    assert torch.allclose(rv, torch.full((4,), 0.9)) and torch.allclose(rm, torch.full((4,), 0.15))


def check_bn_nchw(fn):
    c = GOLDEN["bn_nchw_relu_mean"]
    n, ch, h, w = c["shape"]
    x = from_bits(c["x"], c["shape"])
    sm, sr, out, rm, rv = fn(x, f32(c["gamma"], [ch]), f32(c["beta"], [ch]),
                             f32(c["running_mean"], [ch]), f32(c["running_var"], [ch]),
                             momentum=c["momentum"], eps=c["eps"], var_scale=c["var_scale"],
                             act="relu")
    assert close(out, from_bits(c["out"], [n, ch]), 1.6e-2), "golden out"
    for key, v in (("save_mean", sm), ("save_rstd", sr), ("running_mean_out", rm),
                   ("running_var_out", rv)):
        assert close(v.flatten(), f32(c[key], [ch]), 1e-5), f"golden {key}"
    x = torch.full((3, 2, 2, 2), -4.0, dtype=BF)
    sm, sr, out, rm, rv = fn(x, torch.ones(2), torch.tensor([-0.5, 0.75]), torch.zeros(2),
                             torch.ones(2), momentum=0.1, eps=1e-5, var_scale=1.5, act="relu")
    assert torch.equal(out.float(), torch.tensor([[0.0, 0.75]] * 3)), "relu(beta) on constant channels"


def _exact_gelu_bits(bits):
    """Correctly rounded bf16 GELU(tanh) by mpmath (the GELU table's generator)."""
    import importlib.util
    gen_path = Path(__file__).resolve().parents[1] / "better-benchmark_amd" / "hip_oracles" \
        / "gen_gelu_table.py"
    spec = importlib.util.spec_from_file_location("gen_gelu_table", gen_path)
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    return [gen.to_bf16(gen.gelu_tanh_exact(gen.bf16_value(b))) for b in bits]


def check_gelu_flat(fn):
    # bf16: every 7th finite bit pattern against the exact function at 96
    # bits, rounded to nearest even -- equal but for fp64's own error at a
    # rounding boundary (a handful, one ulp)
    bits = [b for b in range(0, 65536, 7) if (b & 0x7FFF) < 0x7F80]
    x = torch.tensor(bits, dtype=torch.int32).to(torch.int16).view(BF)
    got = fn(x).view(torch.int16).int().tolist()
    want = _exact_gelu_bits(bits)
    off = [(b, g & 0xFFFF, w) for b, g, w in zip(bits, got, want) if (g & 0xFFFF) != w]
    assert len(off) <= 4 and all(abs((g & 0x7FFF) - (w & 0x7FFF)) == 1 for _, g, w in off), \
        f"bf16 vs exact: {[(hex(b), hex(g), hex(w)) for b, g, w in off[:8]]}"
    # specials and closed forms
    sp = torch.tensor([0.0, -0.0, 16.0, 300.0, -16.0, -300.0, float("inf"), float("-inf"),
                       float("nan"), 2.0 ** -20, -(2.0 ** -20)]).to(BF)
    y = fn(sp).float()
    assert y[0] == 0 and not torch.signbit(y[0]) and y[1] == 0 and torch.signbit(y[1])
    assert y[2] == 16.0 and y[3] == 300.0, "gelu(t) = t for large t"
    assert y[4] == 0 and y[5] == 0, "gelu(t) -> 0 for large negative t"
    assert y[6] == float("inf") and torch.isnan(y[7]) and torch.isnan(y[8])
    assert y[9] == 2.0 ** -21 and y[10] == -(2.0 ** -21), "gelu(t) = t / 2 for tiny t"
    # fp32: ATen's own fp64 tanh GELU (an independent implementation) where
    # it does not cancel, and the exact function in the tail
    g = torch.Generator().manual_seed(3)
    xf = torch.randn(20000, generator=g) * 3
    keep = xf > -5
    got = fn(xf)
    want = torch.nn.functional.gelu(xf.double(), approximate="tanh")
    assert torch.allclose(got[keep].double(), want[keep], rtol=1e-6, atol=1e-30), "fp32 vs ATen"
    import mpmath
    for v in (-6.0, -8.5, -12.0):
        t = mpmath.mpf(v)
        u = mpmath.sqrt(2 / mpmath.pi) * (t + mpmath.mpf("0.044715") * t ** 3)
        ex = torch.tensor(float(t / (1 + mpmath.exp(-2 * u))), dtype=torch.float64).float()
        r = fn(torch.tensor([v]))[0]
        assert abs(r - ex) <= 1e-6 * abs(ex) and torch.signbit(r) == torch.signbit(ex), \
            f"fp32 tail gelu({v}) {r.item()} vs {ex.item()}"


def check_transpose(fn):
    g = torch.Generator().manual_seed(5)
    for shape, dtype in (((2, 3, 5, 7), BF), ((4, 49, 128), BF), ((3, 1, 9), torch.float32),
                         ((1, 64, 65), torch.int16), ((6, 6), torch.float32)):
        if dtype == torch.int16:
            x = torch.randint(-32768, 32767, shape, generator=g, dtype=torch.int16)
        else:
            x = torch.randn(shape, generator=g).to(dtype)
        got = fn(x)
        want = x.transpose(-2, -1).contiguous()
        assert got.shape == want.shape and got.is_contiguous(), f"{shape} layout"
        assert torch.equal(got.view(torch.uint8) if got.element_size() == 1 else got, want), \
            f"{shape} values"
    # bit patterns move untouched: NaN payloads and -0 included
    bits = torch.tensor([[0x7FC1, 0xFFFF], [0x8000, 0x7F81]], dtype=torch.int32).to(torch.int16)
    got = fn(bits.view(BF)).view(torch.int16)
    assert torch.equal(got, bits.t().contiguous()), "bit-exact"


def check_row_mean_bf16(fn):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(9, 169, generator=g).to(BF)
    for relu in (False, True):
        got = fn(x, relu=relu)
        rows = x.double().clamp_min(0) if relu else x.double()
        want = [bf16_round(math.fsum(r) / 169) for r in rows.tolist()]
        assert got.float().tolist() == want, f"brute force relu={relu}"
    assert torch.equal(fn(torch.full((3, 13), 2.5, dtype=BF)).float(), torch.full((3,), 2.5))
    assert torch.equal(fn(torch.full((2, 7), -1.0, dtype=BF), relu=True).float(), torch.zeros(2))
    nan_row = torch.tensor([[1.0, float("nan"), -3.0]]).to(BF)
    assert torch.isnan(fn(nan_row, relu=True)).all(), "ReLU keeps NaN"
    mixed = torch.tensor([[4.0, -2.0, 1.0, -7.0]]).to(BF)
    assert fn(mixed, relu=True).item() == 1.25 and fn(mixed).item() == -1.0, "mean(relu(x))"


def check_gelu_erf_bwd(fn):
    g = torch.Generator().manual_seed(13)
    grad = torch.randn(64, 256, generator=g).to(BF)
    x = (2 * torch.randn(64, 256, generator=g)).to(BF)
    y, colsum = fn(grad, x)
    assert y.shape == (64, 256) and y.dtype == BF and colsum.shape == (256,)
    # d against central differences of GELU(t) = t Phi(t) (math.erfc, fp64):
    # y is within one bf16 rounding of grad * d
    def gelu(t):
        return t * math.erfc(-t / math.sqrt(2.0)) / 2
    h = 2.0 ** -12
    for gv, xv, yv in list(zip(grad.flatten().tolist(), x.flatten().tolist(),
                               y.float().flatten().tolist()))[::37]:
        want = gv * (gelu(xv + h) - gelu(xv - h)) / (2 * h)
        assert abs(yv - want) <= 2 ** -8 * abs(want) + 1e-6, (gv, xv, yv, want)
    # colsum: bf16 of the exact (fsum) sum of the returned bf16 y
    cols = y.double().t().tolist()
    assert colsum.tolist() == [bf16_round(math.fsum(c)) for c in cols], "brute-force column sum"
    # closed forms: d(0) = 1/2, d -> 1 and 0 in the tails, inf / NaN -> NaN
    gg = torch.tensor([[1.5, -3.0, 2.0, 7.0, -1.0, 5.0, 2.0, 1.0]]).to(BF)
    xx = torch.tensor([[0.0, -0.0, 20.0, 1e4, -20.0, -1e4, float("inf"), float("nan")]]).to(BF)
    yy, cs = fn(gg, xx)
    assert yy.float()[0, :6].tolist() == [0.75, -1.5, 2.0, 7.0, 0.0, 0.0]
    assert torch.isnan(yy.float()[0, 6:]).all() and torch.isnan(cs[6:]).all()
    # zero rows: zero column sums
    empty = torch.zeros(0, 16, dtype=BF)
    ye, ce = fn(empty, empty)
    assert ye.shape == (0, 16) and torch.equal(ce, torch.zeros(16))


def _rne_bf16_bits(v: float) -> int:
    """fp32 value -> bf16 bits by hand: round to nearest, ties to even."""
    import struct
    u = struct.unpack("<I", struct.pack("<f", v))[0]
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return None  # NaN: any NaN
    lower = u & 0xFFFF
    hi = u >> 16
    if lower > 0x8000 or (lower == 0x8000 and hi & 1):
        hi += 1
    return hi & 0xFFFF


CHECKS = {
    "row_mean": (check_row_mean, ref.row_mean),
    "bias_gelu": (check_bias_gelu, ref.bias_gelu_nchw_to_nhwc),
    "masked_softmax": (check_masked_softmax, ref.scaled_masked_softmax),
    "residual_layernorm": (check_residual_layernorm, ref.residual_layernorm),
    "rmsnorm": (check_rmsnorm, ref.rmsnorm),
    "batchnorm": (check_batchnorm, ref.batchnorm_train),
    "spatial_mean": (check_spatial_mean, ref.spatial_mean_nhwc),
    "bias_softmax": (check_bias_softmax, ref.scaled_bias_softmax),
    "rmsnorm_ex": (check_rmsnorm_ex, ref.rmsnorm_ex),
    "bn_nhwc": (check_bn_nhwc, ref.batchnorm_nhwc_act_pad),
    "bn_nchw": (check_bn_nchw, ref.batchnorm_nchw_act_mean),
    "gelu_flat": (check_gelu_flat, ref.gelu_tanh),
    "transpose": (check_transpose, ref.transpose_last2),
    "row_mean_bf16": (check_row_mean_bf16, ref.row_mean_bf16),
    "gelu_erf_bwd": (check_gelu_erf_bwd, ref.gelu_erf_bwd_colsum),
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


def _spatial_mean_wrong_divisor(x):
    p = x.shape[2] * x.shape[3]
    return (ref.spatial_mean_nhwc(x).float() * p / (p - 1)).to(BF)


def _bias_softmax_groups_reversed(x, bias, scale, heads):
    return ref.scaled_bias_softmax(x, bias.flip(0).contiguous(), scale, heads)


def _rmsnorm_ex_t5_order_dropped(x, g, eps, *, residual=None, scale=1.0, mode=0):
    return ref.rmsnorm_ex(x, g, eps, residual=residual, scale=scale, mode=0)


def _rmsnorm_ex_no_residual(x, g, eps, *, residual=None, scale=1.0, mode=0):
    return ref.rmsnorm_ex(x, g, eps, residual=None, scale=scale, mode=mode)


def _bn_nhwc_pad_top_left(x, *a, **k):
    sm, sr, out, rm, rv = ref.batchnorm_nhwc_act_pad(x, *a, **k)
    return sm, sr, out.roll((1, 1), (2, 3)).contiguous(memory_format=torch.channels_last), rm, rv


def _bn_nhwc_true_bessel(x, g, b, rm, rv, *, var_scale, **k):
    n = x.numel() / x.shape[1]
    return ref.batchnorm_nhwc_act_pad(x, g, b, rm, rv, var_scale=n / (n - 1), **k)


def _bn_nchw_mean_before_relu(x, *a, act=None, **k):
    return ref.batchnorm_nchw_act_mean(x, *a, act=None, **k)


def _gelu_erf_form(x):
    return torch.nn.functional.gelu(x.double()).to(x.dtype)


def _gelu_no_cubic(x):
    return (0.5 * x.double() * (1 + torch.tanh(0.7978845608028654 * x.double()))).to(x.dtype)


def _transpose_leading_dims(x):
    return ref.transpose_last2(x.transpose(0, 1).contiguous()) if x.dim() > 2 else \
        ref.transpose_last2(x).t().contiguous()


def _transpose_reshape_only(x):
    return x.reshape(*x.shape[:-2], x.shape[-1], x.shape[-2]).clone()


def _row_mean_relu_after(x, *, relu=False):
    m = ref.row_mean_bf16(x)
    return m.clamp_min(0) if relu else m


def _row_mean_wrong_divisor(x, *, relu=False):
    return (ref.row_mean_bf16(x, relu=relu).double() * x.shape[1] / (x.shape[1] - 1)).to(BF)


def _gelu_bwd_cdf_only(grad, x):
    """d = Phi(t): the t phi(t) term dropped."""
    d = torch.special.ndtr(x.double())
    y = (grad.double() * d).to(BF)
    return y, y.double().sum(0).to(BF).float()


def _gelu_bwd_sum_unrounded(grad, x):
    """The column sum of grad * d before y's bf16 rounding."""
    y, _ = ref.gelu_erf_bwd_colsum(grad, x)
    exact = grad.float() * ref.gelu_erf_grad(x)
    return y, exact.double().sum(0).to(BF).float()


def _gelu_bwd_unscaled_erf(grad, x):
    """Phi(t) taken as (1 + erf(t)) / 2, without the 1 / sqrt 2."""
    t = x.double()
    d = 0.5 * (1 + torch.erf(t)) + t * torch.exp(-0.5 * t * t) / math.sqrt(2 * math.pi)
    y = (grad.double() * d).to(BF)
    return y, y.double().sum(0).to(BF).float()


MUTANTS = [
    ("gelu_erf_bwd", _gelu_bwd_cdf_only),
    ("gelu_erf_bwd", _gelu_bwd_sum_unrounded),
    ("gelu_erf_bwd", _gelu_bwd_unscaled_erf),
    ("gelu_flat", _gelu_erf_form),
    ("gelu_flat", _gelu_no_cubic),
    ("transpose", _transpose_leading_dims),
    ("transpose", _transpose_reshape_only),
    ("row_mean_bf16", _row_mean_relu_after),
    ("row_mean_bf16", _row_mean_wrong_divisor),
    ("spatial_mean", _spatial_mean_wrong_divisor),
    ("bias_softmax", _bias_softmax_groups_reversed),
    ("rmsnorm_ex", _rmsnorm_ex_t5_order_dropped),
    ("rmsnorm_ex", _rmsnorm_ex_no_residual),
    ("bn_nhwc", _bn_nhwc_pad_top_left),
    ("bn_nhwc", _bn_nhwc_true_bessel),
    ("bn_nchw", _bn_nchw_mean_before_relu),
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


def test_oracle_matches_family_repros():
    """The oracle's family functions against the family repro modules (eager
    ATen, the reference graphs' op order) on small inputs of each family's
    structure."""
    from conftest import CANONICAL
    from oracle_harness import get_repro_instance
    g = torch.Generator().manual_seed(21)
    x = torch.randn(3, 40, 5, 6, generator=g).to(BF).contiguous(memory_format=torch.channels_last)
    want = get_repro_instance(CANONICAL / "mean_c9e1a8113328")(x)
    assert close(ref.spatial_mean_nhwc(x), want, 1.6e-2)
    x, r = torch.randn(6, 64, generator=g).to(BF), torch.randn(2, 3, 64, generator=g).to(BF)
    gm = torch.randn(64, generator=g).to(BF)
    want = get_repro_instance(CANONICAL / "mean_4462ce967d63")(x, r, gm, [2, 3, 64], [6, 64])
    y, _ = ref.rmsnorm_ex(x, gm, 1e-6, residual=r.view(6, 64), scale=0.04419417382415922, mode=1)
    assert close(y, want, 1.6e-2) and exact_fraction(y, want) > 0.97
    x, bias = torch.randn(8, 5, 12, generator=g).to(BF), torch.randn(2, 1, 5, 12, generator=g).to(BF)
    want = get_repro_instance(CANONICAL / "amax_sum_20ccc18dda60")(x, bias, [2, 4, 5, 12], [8, 5, 12])
    assert close(ref.scaled_bias_softmax(x, bias.view(2, 5, 12), 1.0, 4), want, 1.6e-2)
    # decomposed GELU: eager rounds each op to bf16 (the reference harness's
    # allclose 1e-2 holds); in fp32 eager and the oracle agree to fp32 error
    x = (3 * torch.randn(6, 64, generator=g)).to(BF)
    gelu_repro = get_repro_instance(CANONICAL / "pointwise_2d969ac9ad59")
    assert close(ref.gelu_tanh(x), gelu_repro(x, [2, 3, 64], [6, 64]), 1e-2)
    xf = 3 * torch.randn(6, 64, generator=g)
    assert torch.allclose(ref.gelu_tanh(xf), gelu_repro(xf, [2, 3, 64], [-1, 64]),
                          rtol=1e-5, atol=1e-6)
    x = torch.randn(2, 3, 4, 8, generator=g).to(BF)
    want = get_repro_instance(CANONICAL / "pointwise_021e90d9c17d")(x, [2, 24, 2, 2])
    assert torch.equal(ref.transpose_last2(x).view(2, 24, 2, 2), want)
    x = torch.randn(6, 5, 12, generator=g).to(BF)
    want = get_repro_instance(CANONICAL / "amax_sum_fa4cc85fe5ad")(
        x, [2, 3, 5, 12], [2, 3, 5, 12], [6, 5, 12])
    zero = torch.zeros(1, 12, dtype=BF)
    assert close(ref.scaled_masked_softmax(x.reshape(30, 1, 12), zero, 1.0).view(6, 5, 12),
                 want, 1.6e-2)
    grad, x = torch.randn(12, 16, generator=g).to(BF), torch.randn(12, 16, generator=g).to(BF)
    want = get_repro_instance(CANONICAL / "sum_139a3020e8bf")(
        grad, x, [3, 4, 16], [3, 4, 16], [12, 16], [16])
    y, colsum = ref.gelu_erf_bwd_colsum(grad, x)
    assert close(y, want[0], 1.6e-2) and close(y.t(), want[1], 1.6e-2)
    assert close(colsum, want[2], 1e-2)
    x = torch.randn(2, 5, 3, 3, generator=g).to(BF)
    want = get_repro_instance(CANONICAL / "mean_b402ee209d0b")(x, [2, 5])
    assert close(ref.row_mean_bf16(x.reshape(10, 9), relu=True).view(2, 5), want, 1.6e-2)
    for rid, fmt, call in (
            ("var_mean_ceb5c315290a", torch.channels_last,
             lambda x, rm, rv, w, b: ref.batchnorm_nhwc_act_pad(
                 x, w, b, rm, rv, momentum=0.1, eps=1e-3, var_scale=1.00000996502277,
                 act="silu", pad_bottom=1, pad_right=1)),
            ("var_mean_mean_19ffdb35cc67", torch.contiguous_format,
             lambda x, rm, rv, w, b: ref.batchnorm_nchw_act_mean(
                 x, w, b, rm, rv, momentum=0.1, eps=1e-5, var_scale=1.0001594642002871,
                 act="relu"))):
        x = (2 * torch.randn(3, 8, 5, 4, generator=g) + 0.5).to(BF).contiguous(memory_format=fmt)
        rm, rv, w, b = (torch.randn(8, generator=g), torch.rand(8, generator=g) + 0.5,
                        torch.randn(8, generator=g), torch.randn(8, generator=g))
        got = call(x, rm, rv, w, b)
        want = get_repro_instance(CANONICAL / rid)(x, rm.clone(), rv.clone(), w, b)
        for i, (a_, b_) in enumerate(zip(got, want)):
            assert close(a_, b_, 1.6e-2 if b_.dtype == BF else 1e-5), f"{rid} out{i}"
