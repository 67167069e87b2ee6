"""
Canonical repro of the reference family mean_d28c6a07654f
(Mistral-7B-Instruct-v0.3, Qwen3-0.6B): residual add + RMSNorm over the last
dim, eps 1e-06, returning the bf16 sum h and 2 views of y.
Semantics of the reference's
repros/canonical/mean_d28c6a07654f/repro.py:24-38: h = bf16(residual +
view(x)); rstd = rsqrt(mean(h^2) + 1e-06) in fp32; t = bf16(h * rstd), y =
bf16(gamma * t).  The shape points are that dir's shapes.json points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
EPS = 1e-06


def _upcast(t):
    # fp32 for the bf16 sum (the graph's convert_element_type); an fp64 copy
    # of the module (the numerics gate's anchor) stays in fp64.
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[1000, 1024]",
                arg1_1: "bf16[1, 1000, 1024]",
                arg2_1: "bf16[1024]",
                _shape_param_0, _shape_param_1, _shape_param_2):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        add = torch.ops.aten.add.Tensor(arg1_1, view)
        h = _upcast(add)
        ms = torch.ops.aten.mean.dim(torch.ops.aten.pow.Tensor_Scalar(h, 2), [-1], True)
        rstd = torch.ops.aten.rsqrt.default(torch.ops.aten.add.Tensor(ms, EPS))
        t = torch.ops.prims.convert_element_type.default(
            torch.ops.aten.mul.Tensor(h, rstd), arg0_1.dtype)
        out = torch.ops.aten.mul.Tensor(arg2_1, t)
        return (add,
                torch.ops.aten.view.default(out, _shape_param_1),
                torch.ops.aten.view.default(out, _shape_param_2))


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
