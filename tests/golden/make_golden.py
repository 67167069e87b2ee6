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

    doc = {"generator": "tests/golden/make_golden.py",
           "producer": f"torch {torch.__version__} eager ATen CPU kernels",
           "cases": cases}
    OUT.write_text(json.dumps(doc, indent=0, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
