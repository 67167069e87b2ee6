"""
Canonical repro of the reference family var_mean_80e7ff4dee7f (HF Allenai
Longformer-base inference): residual add + LayerNorm, y only.
Semantics of the reference's repros/canonical/var_mean_80e7ff4dee7f/repro.py:23-39:
h = bf16(view(x) + residual); fp32 var_mean (correction 0) over the last
dim; (h - mean) * rsqrt(var + 1e-5) * gamma + beta in fp32; bf16 out.  The
shape point is that dir's shapes.json point (x given flat as [8192, 768]).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
EPS = 1e-05


def _upcast(t):
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[8192, 768]", arg1_1: "bf16[8, 1024, 768]",
                arg2_1: "bf16[768]", arg3_1: "bf16[768]", _shape_param_0):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        h = _upcast(torch.ops.aten.add.Tensor(view, arg1_1))
        var, mean = torch.ops.aten.var_mean.correction(h, [2], correction=0, keepdim=True)
        rstd = torch.ops.aten.rsqrt.default(torch.ops.aten.add.Tensor(var, EPS))
        y = torch.ops.aten.mul.Tensor(torch.ops.aten.sub.Tensor(h, mean), rstd)
        y = torch.ops.aten.add.Tensor(torch.ops.aten.mul.Tensor(y, arg2_1), arg3_1)
        return torch.ops.prims.convert_element_type.default(y, arg0_1.dtype)


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
