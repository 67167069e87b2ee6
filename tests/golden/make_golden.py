"""Write tests/golden/aten_eager_small.json: tiny seeded inputs and the
outputs PyTorch's eager ATen CPU kernels produce for them.

The reference holds no numeric golden vectors for these patterns (its
oracle checks are always in-run eager-vs-oracle comparisons), and the
arithmetic it relies on lives in PyTorch (ATen), a dependency it does not
vendor or pin.  These fixtures pin the CPU oracle (oracle/hipo_ref.c) to
ATen's own results at a fixed version (recorded in the file), independent
of the oracle's code.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
from pathlib import Path

import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "aten_eager_small.json"


def bits(t: torch.Tensor) -> list[int]:
    """bf16 tensor -> list of uint16 bit patterns (row-major)."""
    return (t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF).flatten().tolist()


def floats(t: torch.Tensor) -> list[float]:
    return [float(v) for v in t.contiguous().flatten().tolist()]


def main() -> None:
    g = torch.Generator().manual_seed(2024)
    bf = torch.bfloat16
    cases = {}

    x = torch.randn(5, 37, generator=g)
    cases["row_mean"] = {"x": floats(x), "shape": [5, 37],
                         "out": floats(torch.ops.aten.mean.dim(x, [-1]))}

    x = torch.randn(2, 16, 3, 5, generator=g).to(bf)
    b = (0.1 * torch.randn(16, generator=g)).to(bf)
    y = F.gelu(x + b.view(1, -1, 1, 1), approximate="tanh").contiguous(
        memory_format=torch.channels_last)
    cases["bias_gelu_nhwc"] = {"x": bits(x), "bias": bits(b), "shape": [2, 16, 3, 5],
                               "out_nhwc": bits(y.permute(0, 2, 3, 1))}

    x = torch.randn(3, 6, 20, generator=g).to(bf)
    mask = torch.triu(torch.full((6, 20), float("-inf")), 1).to(bf)
    y = torch.softmax(x * 0.125 + mask, -1)
    cases["masked_softmax"] = {"x": bits(x), "mask": bits(mask), "shape": [3, 6, 20],
                               "scale": 0.125, "out": bits(y)}

    x = torch.randn(4, 48, generator=g).to(bf)
    r = torch.randn(4, 48, generator=g).to(bf)
    gm = (1 + 0.1 * torch.randn(48, generator=g)).to(bf)
    bt = (0.1 * torch.randn(48, generator=g)).to(bf)
    h = x + r
    hf = h.float()
    var, mean = torch.var_mean(hf, -1, correction=0, keepdim=True)
    rstd = torch.rsqrt(var + 1e-5)
    y = ((hf - mean) * rstd * gm.float() + bt.float()).to(bf)
    cases["residual_layernorm"] = {
        "x": bits(x), "residual": bits(r), "gamma": bits(gm), "beta": bits(bt),
        "shape": [4, 48], "eps": 1e-5, "h": bits(h), "y": bits(y),
        "mean": floats(mean.squeeze(-1)), "rstd": floats(rstd.squeeze(-1))}

    y = F.rms_norm(x, [48], gm, 1e-5)
    rs = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-5)
    cases["rmsnorm"] = {"x": bits(x), "gamma": bits(gm), "shape": [4, 48], "eps": 1e-5,
                        "y": bits(y), "rstd": floats(rs)}

    x = torch.randn(3, 4, 5, 6, generator=g) * 2 + 0.5
    w = 1 + 0.1 * torch.randn(4, generator=g)
    bb = 0.1 * torch.randn(4, generator=g)
    rm, rv = torch.zeros(4), torch.ones(4)
    out, sm, si = torch.ops.aten.native_batch_norm(x, w, bb, rm, rv, True, 0.1, 1e-5)
    cases["batchnorm_train"] = {
        "x": floats(x), "gamma": floats(w), "beta": floats(bb), "shape": [3, 4, 5, 6],
        "momentum": 0.1, "eps": 1e-5, "y_relu": floats(torch.relu(out)),
        "save_mean": floats(sm), "save_invstd": floats(si),
        "running_mean": floats(rm), "running_var": floats(rv)}

    # --- corpus families (appended: the cases above keep their inputs) ---
    x = (torch.randn(2, 24, 3, 5, generator=g) + 0.3).to(bf).contiguous(
        memory_format=torch.channels_last)
    cases["spatial_mean_nhwc"] = {"x_nhwc": bits(x.permute(0, 2, 3, 1)), "shape": [2, 24, 3, 5],
                                  "out": bits(torch.ops.aten.mean.dim(x, [2, 3], True))}

    x = torch.randn(6, 4, 12, generator=g).to(bf)          # 2 bias groups x 3 heads
    bias = torch.randn(2, 4, 12, generator=g).to(bf)
    s4 = torch.ops.aten.add.Tensor(torch.ops.aten.mul.Tensor(x, 0.5).view(2, 3, 4, 12),
                                   bias.view(2, 1, 4, 12))
    y = torch.softmax(s4.float(), -1).to(bf).view(6, 4, 12)
    cases["bias_softmax"] = {"x": bits(x), "bias": bits(bias), "shape": [6, 4, 12], "heads": 3,
                             "scale": 0.5, "out": bits(y)}

    x = torch.randn(6, 32, generator=g).to(bf)
    r = torch.randn(6, 32, generator=g).to(bf)
    gm = (1 + 0.1 * torch.randn(32, generator=g)).to(bf)
    h = r + x
    rs = torch.rsqrt(h.float().pow(2).mean(-1, keepdim=True) + 1e-6)
    t5 = (gm * (h.float() * rs).to(bf)) * 0.04419417382415922
    cases["rmsnorm_t5"] = {"x": bits(x), "residual": bits(r), "gamma": bits(gm), "shape": [6, 32],
                           "eps": 1e-6, "scale": 0.04419417382415922, "y": bits(t5),
                           "rstd": floats(rs.squeeze(-1)),
                           "y_residual_rms_norm": bits(F.rms_norm(h, [32], gm, 1e-6))}

    def bn_bf16(x, rm, rv, w, b, eps, var_scale):
        var, mean = torch.var_mean(x.float(), [0, 2, 3], correction=0, keepdim=True)
        rstd = torch.rsqrt(var + eps)
        t = ((x - mean) * rstd * w.view(-1, 1, 1) + b.view(-1, 1, 1)).to(bf)
        rm2 = mean.flatten() * 0.1 + rm * 0.9
        rv2 = var.flatten() * var_scale * 0.1 + rv * 0.9
        return mean, rstd, t, rm2, rv2

    x = (2 * torch.randn(3, 8, 4, 5, generator=g) + 0.5).to(bf).contiguous(
        memory_format=torch.channels_last)
    rm, rv = torch.randn(8, generator=g), torch.rand(8, generator=g) + 0.5
    w, b = 1 + 0.1 * torch.randn(8, generator=g), 0.1 * torch.randn(8, generator=g)
    mean, rstd, t, rm2, rv2 = bn_bf16(x, rm, rv, w, b, 1e-3, 1.25)
    tf = t.float()
    silu = (tf / (1 + torch.exp(-tf))).to(bf)
    out = torch.ops.aten.constant_pad_nd.default(silu, [0, 1, 0, 1], 0.0)
    cases["bn_nhwc_silu_pad"] = {
        "x_nhwc": bits(x.permute(0, 2, 3, 1)), "shape": [3, 8, 4, 5], "running_mean": floats(rm),
        "running_var": floats(rv), "gamma": floats(w), "beta": floats(b), "eps": 1e-3,
        "momentum": 0.1, "var_scale": 1.25, "pad": [1, 1], "save_mean": floats(mean),
        "save_rstd": floats(rstd), "out_nhwc": bits(out.permute(0, 2, 3, 1)),
        "running_mean_out": floats(rm2), "running_var_out": floats(rv2)}

    x = (2 * torch.randn(5, 8, 3, 3, generator=g) + 0.5).to(bf)
    rm, rv = torch.randn(8, generator=g), torch.rand(8, generator=g) + 0.5
    w, b = 1 + 0.1 * torch.randn(8, generator=g), 0.1 * torch.randn(8, generator=g)
    mean, rstd, t, rm2, rv2 = bn_bf16(x, rm, rv, w, b, 1e-5, 1.5)
    out = torch.ops.aten.mean.dim(torch.relu(t), [2, 3])
    cases["bn_nchw_relu_mean"] = {
        "x": bits(x), "shape": [5, 8, 3, 3], "running_mean": floats(rm), "running_var": floats(rv),
        "gamma": floats(w), "beta": floats(b), "eps": 1e-5, "momentum": 0.1, "var_scale": 1.5,
        "save_mean": floats(mean), "save_rstd": floats(rstd), "out": bits(out),
        "running_mean_out": floats(rm2), "running_var_out": floats(rv2)}

    doc = {"generator": "tests/golden/make_golden.py",
           "producer": f"torch {torch.__version__} eager ATen CPU kernels",
           "cases": cases}
    OUT.write_text(json.dumps(doc, indent=0, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
