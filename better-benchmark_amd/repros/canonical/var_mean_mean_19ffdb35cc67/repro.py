"""
Canonical repro of the reference family var_mean_mean_19ffdb35cc67
(torchbench shufflenet_v2_x1_0 training): BatchNorm training forward of an
NCHW bf16 activation with fp32 statistics, ReLU, and the mean over H, W.
Semantics of the reference's repros/canonical/var_mean_mean_19ffdb35cc67/repro.py:23-54:
mean, var = var_mean(fp32(x), [0, 2, 3], correction=0); rstd = rsqrt(var + 1e-5);
r = relu(bf16(((x - mean) * rstd) * gamma + beta)); out = mean(r, [2, 3]) (bf16);
running_mean <- mean * 0.1 + running_mean * 0.9 and
running_var <- var * 1.0001594642002871 * 0.1 + running_var * 0.9, in place.
Inputs in the graph's order: x, running_mean, running_var, gamma, beta.
Returns (mean, rstd, out, running_mean, running_var).  Casts are "at least
fp32" / "back to x's dtype" (fp64 throughout in the numerics gate's copy).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
EPS = 1e-05
MOMENTUM = 0.1
KEEP = 0.9
VAR_SCALE = 1.0001594642002871
aten = torch.ops.aten


def _upcast(t):
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


def _per_channel(v):
    return aten.unsqueeze.default(aten.unsqueeze.default(v, -1), -1)


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[128, 1024, 7, 7]", arg1_1: "f32[1024]",
                arg2_1: "f32[1024]", arg3_1: "f32[1024]", arg4_1: "f32[1024]"):
        var, mean = aten.var_mean.correction(_upcast(arg0_1), [0, 2, 3], correction=0,
                                             keepdim=True)
        rstd = aten.rsqrt.default(aten.add.Tensor(var, EPS))
        norm = aten.mul.Tensor(aten.sub.Tensor(arg0_1, mean), rstd)
        affine = aten.add.Tensor(aten.mul.Tensor(norm, _per_channel(arg3_1)), _per_channel(arg4_1))
        relu = aten.relu.default(torch.ops.prims.convert_element_type.default(affine, arg0_1.dtype))
        out = aten.mean.dim(relu, [2, 3])
        new_mean = aten.add.Tensor(aten.mul.Tensor(aten.squeeze.dims(mean, [0, 2, 3]), MOMENTUM),
                                   aten.mul.Tensor(arg1_1, KEEP))
        new_var = aten.add.Tensor(
            aten.mul.Tensor(aten.mul.Tensor(aten.squeeze.dims(var, [0, 2, 3]), VAR_SCALE), MOMENTUM),
            aten.mul.Tensor(arg2_1, KEEP))
        running_mean = aten.copy_.default(arg1_1, new_mean)
        running_var = aten.copy_.default(arg2_1, new_var)
        return (mean, rstd, out, running_mean, running_var)


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
