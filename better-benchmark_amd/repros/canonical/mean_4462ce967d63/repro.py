"""
Canonical repro of the reference family mean_4462ce967d63 (HF T5 / T5Small
inference): residual add + T5-style RMSNorm in the HF op order.
Semantics of the reference's repros/canonical/mean_4462ce967d63/repro.py:23-38:
h = bf16(residual + x); rstd = rsqrt(mean(h^2) + 1e-6) in fp32;
y = bf16(bf16(gamma * bf16(h * rstd)) * 0.04419417382415922); the shape
point is that dir's shapes.json point (x given flat as [8192, 512]).
Casts are "at least fp32" / "back to the input dtype", so the fp64 copy of
the numerics gate computes the whole graph in fp64.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
EPS = 1e-06
SCALE = 0.04419417382415922


def _upcast(t):
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[8192, 512]", arg1_1: "bf16[8, 1024, 512]",
                arg2_1: "bf16[512]", _shape_param_0, _shape_param_1):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        add = torch.ops.aten.add.Tensor(arg1_1, view)
        sq = torch.ops.aten.pow.Tensor_Scalar(_upcast(add), 2)
        mean = torch.ops.aten.mean.dim(sq, [-1], True)
        rsqrt = torch.ops.aten.rsqrt.default(torch.ops.aten.add.Tensor(mean, EPS))
        normed = torch.ops.prims.convert_element_type.default(
            torch.ops.aten.mul.Tensor(add, rsqrt), arg0_1.dtype)
        scaled = torch.ops.aten.mul.Tensor(torch.ops.aten.mul.Tensor(arg2_1, normed), SCALE)
        return torch.ops.aten.view.default(scaled, _shape_param_1)


def _default_make_inputs():
    configs = load_shape_configs(__file__)
    if not configs:
        raise RuntimeError("no shapes.json next to this repro")
    return make_inputs_from_config(next(iter(configs.values())))


def make_inputs(shape_config=None):
    """Inputs for a shape config (default: the first shapes.json point)."""
    if shape_config is not None:
        return make_inputs_from_config(shape_config)
    return _default_make_inputs()


if __name__ == "__main__":
    benchmark_repro(__file__, Repro, make_inputs)
