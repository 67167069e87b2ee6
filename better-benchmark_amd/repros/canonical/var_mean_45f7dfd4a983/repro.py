"""
Canonical repro of the reference family var_mean_45f7dfd4a983
(AlbertForMaskedLM, BartForCausalLM, DistillGPT2, PLBartForCausalLM and 1
more): residual add + LayerNorm over the last dim, eps 1e-12, returning y
and an [R, C] view of it.
Semantics of the reference's
repros/canonical/var_mean_45f7dfd4a983/repro.py:24-40: h = bf16(residual +
view(x)) (arg1_1 + arg0_1 viewed 3-D); fp32 var_mean (correction 0) of h
over the last dim; rsqrt(var + 1e-12); (h - mean) * rstd * gamma + beta in
fp32; bf16 out.  The shape points are that dir's shapes.json points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
EPS = 1e-12


def _upcast(t):
    # fp32 for the bf16 sum (the graph's convert_element_type); an fp64 copy
    # of the module (the numerics gate's anchor) stays in fp64.
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[4096, 4096]",
                arg1_1: "bf16[8, 512, 4096]",
                arg2_1: "bf16[4096]",
                arg3_1: "bf16[4096]",
                _shape_param_0, _shape_param_1):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        add = torch.ops.aten.add.Tensor(arg1_1, view)
        h = _upcast(add)
        var, mean = torch.ops.aten.var_mean.correction(h, [2], correction=0, keepdim=True)
        rstd = torch.ops.aten.rsqrt.default(torch.ops.aten.add.Tensor(var, EPS))
        y = torch.ops.aten.mul.Tensor(torch.ops.aten.sub.Tensor(h, mean), rstd)
        y = torch.ops.aten.add.Tensor(torch.ops.aten.mul.Tensor(y, arg2_1), arg3_1)
        out = torch.ops.prims.convert_element_type.default(y, arg0_1.dtype)
        return (out, torch.ops.aten.view.default(out, _shape_param_1))


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
