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


def check_cast(fn):
    # bf16 -> fp32: every bf16 pattern, its bits in the high half
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(BF)
    y = fn(x, torch.float32)
    assert y.dtype == torch.float32
    want = ((x.view(torch.int16).to(torch.int64) & 0xFFFF) << 16).to(torch.int32)
    assert torch.equal(y.view(torch.int32), want), "bf16 -> fp32 is exact"
    # fp32 -> bf16: by hand (nearest even) on ties, near-ties, subnormals,
    # overflow to inf, and ATen's own cast on random patterns
    vals = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 1.0 + 2 ** -8 + 2 ** -20,
            3.3895313892515355e38, 3.4028234663852886e38, 1e-40, -1e-42, 2 ** -133,
            2 ** -134, 0.0, -0.0, float("inf"), -float("inf"), 65504.0, 0.1, -7.3e-5]
    got = fn(torch.tensor(vals), BF).view(torch.int16).tolist()
    for v, gb in zip(vals, got):
        assert (gb & 0xFFFF) == _rne_bf16_bits(v), (v, hex(gb & 0xFFFF))
    g = torch.Generator().manual_seed(9)
    bits = torch.randint(-(2 ** 31), 2 ** 31 - 1, (20000,), generator=g, dtype=torch.int64)
    xf = bits.to(torch.int32).view(torch.float32)
    yb = fn(xf, BF)
    want = xf.to(BF)
    nan = torch.isnan(want.float())
    assert torch.equal(torch.isnan(yb.float()), nan)
    assert torch.equal(yb.view(torch.int16)[~nan], want.view(torch.int16)[~nan]), "vs ATen"
    # strides kept (channels-last in, channels-last out)
    xc = torch.randn(2, 5, 3, 4).to(memory_format=torch.channels_last)
    yc = fn(xc, BF)
    assert yc.stride() == xc.stride() and torch.equal(yc, xc.to(BF))


def _bn_eager(x, mean, var, w, b, eps, act, residual=None, second=None):
    """The families' ATen graph on the CPU (sub, add eps, sqrt, reciprocal,
    mul, mul, add, bf16 cast, then the epilogue's bf16 ops)."""
    def affine(x, mean, var, w, b):
        inv = torch.reciprocal(torch.sqrt(var.float() + eps)) * 1
        sh = (-1, 1, 1)
        t = (x - mean.float().reshape(sh)) * inv.reshape(sh)
        return ((t * w.reshape(sh)) + b.reshape(sh)).to(BF)
    t = affine(x, mean, var, w, b)
    if second is not None:
        t = t + affine(*second)
    if residual is not None:
        t = t + residual
    if act == "relu":
        t = torch.relu(t)
    elif act == "relu6":
        t = torch.clamp_max(torch.clamp_min(t.float(), 0.0), 6.0).to(BF)
    return t


def _bn_anchor(x, mean, var, w, b, eps, act, residual=None, second=None):
    """The families' graph as its fp64 evaluation makes it."""
    import numpy as np

    def affine(x, mean, var, w, b):
        v = var.float().numpy()
        inv = torch.from_numpy(np.float32(1) / np.sqrt(v + np.float32(eps))).double()
        sh = (-1, 1, 1)
        t = (x.double() - mean.double().reshape(sh)) * inv.reshape(sh)
        t = t * w.double().reshape(sh) + b.double().reshape(sh)
        return t.float().to(BF)
    t = affine(x, mean, var, w, b)
    if second is not None:
        t = t + affine(*second)
    if residual is not None:
        t = t + residual
    if act == "relu":
        t = torch.relu(t)
    elif act == "relu6":
        t = torch.clamp_max(torch.clamp_min(t.float(), 0.0), 6.0).to(BF)
    return t


def _bn_params(c, gen, *, var_lo=0.05):
    mean = (torch.randn(c, generator=gen) * 0.5).to(BF)
    var = (torch.rand(c, generator=gen) * 2 + var_lo).to(BF)
    w = (torch.randn(c, generator=gen)).to(BF)
    b = (torch.randn(c, generator=gen) * 0.3).to(BF)
    return mean, var, w, b


def check_bn_infer(fn):
    f32 = lambda v: torch.tensor(v, dtype=torch.float32)  # noqa: E731
    one = lambda v, c=1: torch.full((c,), v).to(BF)  # noqa: E731
    # closed forms: x == mean leaves the bias; var + eps = 4 halves x - mean
    x = torch.full((1, 1, 2, 2), 1.5).to(BF)
    y = fn(x, one(1.5), one(3.75), one(-2.0), one(0.625), eps=0.25, act="none")
    assert torch.equal(y.float(), torch.full((1, 1, 2, 2), 0.625))
    y = fn(torch.full((1, 1, 1, 2), 5.5).to(BF), one(1.5), one(3.75), one(3.0), one(-1.0),
           eps=0.25, act="none")
    assert torch.equal(y.float(), torch.full((1, 1, 1, 2), 5.0)), "(4 * 0.5) * 3 - 1"
    # eps inside the sqrt: var 0, eps 0.25 -> inv 2
    y = fn(torch.full((1, 1, 1, 1), 1.0).to(BF), one(0.0), one(0.0), one(1.0), one(0.0),
           eps=0.25, act="none")
    assert y.float().item() == 2.0
    # the affine is rounded to bf16 before the residual add:
    # (1 + 2^-7)(1 + 3 * 2^-7) = 1 + 2^-5 + 3 * 2^-14 -> bf16 1 + 2^-5; - 1 -> 2^-5
    y = fn(torch.full((1, 1, 1, 1), 1 + 2 ** -7).to(BF), one(0.0), one(0.75), one(1 + 3 * 2 ** -7),
           one(0.0), eps=0.25, act="none", residual=torch.full((1, 1, 1, 1), -1.0).to(BF))
    assert y.float().item() == 2 ** -5, y.float().item()
    # two affines, each rounded, then their sum rounded, then relu
    y = fn(torch.full((1, 1, 1, 1), 1 + 2 ** -7).to(BF), one(0.0), one(0.75), one(1 + 3 * 2 ** -7),
           one(0.0), eps=0.25, act="relu",
           second=(torch.full((1, 1, 1, 1), -4.0).to(BF), one(0.0), one(0.75), one(1.0),
                   one(0.0)))
    assert y.float().item() == 0.0
    # relu6 clamps at 6 and keeps NaN; relu keeps NaN and zeroes negatives
    xs = torch.tensor([[-3.0, 2.5, 7.0, float("nan")]]).reshape(1, 1, 1, 4).to(BF)
    p = (one(0.0), one(0.75), one(1.0), one(0.0))
    y6 = fn(xs, *p, eps=0.25, act="relu6").float().flatten()
    assert y6[:3].tolist() == [0.0, 2.5, 6.0] and torch.isnan(y6[3])
    y1 = fn(xs, *p, eps=0.25, act="relu").float().flatten()
    assert y1[:3].tolist() == [0.0, 2.5, 7.0] and torch.isnan(y1[3])
    # channel placement in both layouts: x = 0, mean = -c, inv = 1 -> y = c
    c = 12
    ch = torch.arange(c, dtype=torch.float32)
    for fmt in (torch.contiguous_format, torch.channels_last):
        x0 = torch.zeros(2, c, 3, 5).to(BF).to(memory_format=fmt)
        y = fn(x0, (-ch).to(BF), torch.full((c,), 0.75).to(BF), torch.ones(c).to(BF),
               torch.zeros(c).to(BF), eps=0.25, act="none")
        assert y.stride() == x0.stride()
        assert torch.equal(y.float(), ch.reshape(1, c, 1, 1).expand(2, c, 3, 5)), fmt
    # vs the graph's fp64 evaluation (the harness's numerics anchor: inv in
    # fp32, by numpy's IEEE sqrt and division; the element ops by ATen in
    # fp64; the bf16 casts through fp32) on random data: layouts, odd C,
    # every epilogue
    gen = torch.Generator().manual_seed(23)
    for (n, c, h, w), fmt in (((2, 24, 7, 7), torch.contiguous_format),
                              ((3, 20, 5, 4), torch.channels_last),
                              ((1, 13, 3, 3), torch.channels_last),
                              ((2, 9, 4, 4), torch.contiguous_format)):
        xr = (torch.randn(n, c, h, w, generator=gen) * 2).to(BF).to(memory_format=fmt)
        rr = torch.randn(n, c, h, w, generator=gen).to(BF).to(memory_format=fmt)
        x2 = (torch.randn(n, c, h, w, generator=gen) * 2).to(BF).to(memory_format=fmt)
        pa, pb = _bn_params(c, gen), _bn_params(c, gen)
        for act, kw in (("relu", {}), ("none", {}), ("none", {"residual": rr}),
                        ("relu6", {}), ("relu", {"residual": rr}),
                        ("relu", {"second": (x2, *pb)})):
            for eps in (1e-3, 1e-5):
                got = fn(xr, *pa, eps=eps, act=act, **kw)
                want = _bn_anchor(xr, *pa, eps, act, **kw)
                assert got.stride() == xr.stride()
                torch.testing.assert_close(got, want, rtol=0, atol=0, equal_nan=True,
                                           msg=f"{(n, c, h, w)} {fmt} {act} {list(kw)} {eps}")


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
    "cast": (check_cast, ref.cast_storage),
    "bn_infer": (check_bn_infer, ref.bn_infer_act),
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


def _cast_truncates(x, dtype):
    """fp32 -> bf16 by dropping the low half (round toward zero)."""
    if x.dtype == torch.float32 and dtype == BF:
        return (x.contiguous().view(torch.int32) >> 16).to(torch.int16).view(BF).reshape(x.shape)
    return ref.cast_storage(x, dtype)


def _cast_ties_away(x, dtype):
    """fp32 -> bf16 with ties rounded away from zero."""
    if x.dtype == torch.float32 and dtype == BF:
        u = x.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        r = ((u + 0x8000) >> 16) & 0xFFFF
        nan = torch.isnan(x.contiguous())
        r = torch.where(nan, torch.full_like(r, 0x7FC0), r)
        return r.to(torch.int32).to(torch.int16).view(BF).reshape(x.shape)
    return ref.cast_storage(x, dtype)


def _bn_infer_unrounded_residual(x, mean, var, w, b, *, eps, act="none", residual=None,
                                 second=None):
    """The affine kept in fp32 through the residual add (one rounding)."""
    if residual is None:
        return ref.bn_infer_act(x, mean, var, w, b, eps=eps, act=act, second=second)
    sh = (-1, 1, 1)
    inv = torch.reciprocal(torch.sqrt(var.float() + eps)).reshape(sh)
    t = ((x.float() - mean.float().reshape(sh)) * inv) * w.float().reshape(sh) + b.float().reshape(sh)
    t = (t + residual.float()).to(BF)
    return torch.relu(t) if act == "relu" else t


def _bn_infer_eps_outside(x, mean, var, w, b, *, eps, act="none", residual=None, second=None):
    """1 / (sqrt(var) + eps) instead of 1 / sqrt(var + eps)."""
    return _bn_eager_with_inv(x, mean, var, w, b, eps, act, residual, second,
                              lambda v: 1.0 / (torch.sqrt(v) + eps))


def _bn_eager_with_inv(x, mean, var, w, b, eps, act, residual, second, inv_of):
    def affine(x, mean, var, w, b):
        sh = (-1, 1, 1)
        t = (x.float() - mean.float().reshape(sh)) * inv_of(var.float()).reshape(sh)
        return (t * w.float().reshape(sh) + b.float().reshape(sh)).to(BF)
    t = affine(x, mean, var, w, b)
    if second is not None:
        t = t + affine(*second)
    if residual is not None:
        t = t + residual
    if act == "relu":
        t = torch.relu(t)
    elif act == "relu6":
        t = torch.clamp(t.float(), 0.0, 6.0).to(BF)
    return t


def _bn_infer_nchw_channel_always(x, mean, var, w, b, *, eps, act="none", residual=None,
                                  second=None):
    """Channel of storage element i taken as (i / HW) % C whatever the layout."""
    def as_nchw(t):
        return torch.as_strided(t, tuple(t.shape), tuple(torch.empty(t.shape).stride()))
    sec = None if second is None else (as_nchw(second[0]), *second[1:])
    res = None if residual is None else as_nchw(residual)
    y = ref.bn_infer_act(as_nchw(x), mean, var, w, b, eps=eps, act=act, residual=res, second=sec)
    return torch.as_strided(y, tuple(x.shape), tuple(x.stride()))


def _bn_infer_relu6_as_relu(x, mean, var, w, b, *, eps, act="none", residual=None,
                            second=None):
    """ReLU6's upper clamp dropped."""
    act = "relu" if act == "relu6" else act
    return ref.bn_infer_act(x, mean, var, w, b, eps=eps, act=act, residual=residual,
                            second=second)


MUTANTS = [
    ("bn_infer", _bn_infer_unrounded_residual),
    ("bn_infer", _bn_infer_eps_outside),
    ("bn_infer", _bn_infer_nchw_channel_always),
    ("bn_infer", _bn_infer_relu6_as_relu),
    ("cast", _cast_truncates),
    ("cast", _cast_ties_away),
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
