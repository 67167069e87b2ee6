"""
Canonical repro of the reference family var_mean_ceb5c315290a (timm
tf_efficientnet_b0 training): BatchNorm training forward of a channels-last
bf16 activation with fp32 statistics, SiLU, and a zero pad of the bottom and
right border.
Semantics of the reference's repros/canonical/var_mean_ceb5c315290a/repro.py:27-58:
mean, var = var_mean(fp32(x), [0, 2, 3], correction=0); rstd = rsqrt(var + 1e-3);
t = bf16(((x - mean) * rstd) * gamma + beta); y = bf16(t / (1 + exp(-t)));
out = pad(y, [0, 1, 0, 1]) (channels-last);
running_mean <- mean * 0.1 + running_mean * 0.9 and
running_var <- var * 1.00000996502277 * 0.1 + running_var * 0.9, in place (the
constant is the graph's Bessel factor at its first shape point and is kept
for every point).  Inputs in the graph's order: x, running_mean, running_var,
gamma, beta.  Returns (mean, rstd, out, running_mean, running_var).
Casts are "at least fp32" / "back to x's dtype", so the fp64 copy of the
numerics gate computes the whole graph in fp64.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
EPS = 1e-3
MOMENTUM = 0.1
KEEP = 0.9
VAR_SCALE = 1.00000996502277
aten = torch.ops.aten


def _upcast(t):
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


def _down(t, dtype):
    return torch.ops.prims.convert_element_type.default(t, dtype)


def _per_channel(v):
    return aten.unsqueeze.default(aten.unsqueeze.default(v, -1), -1)


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[128, 240, 28, 28]", arg1_1: "f32[240]",
                arg2_1: "f32[240]", arg3_1: "f32[240]", arg4_1: "f32[240]"):
        var, mean = aten.var_mean.correction(_upcast(arg0_1), [0, 2, 3], correction=0,
                                             keepdim=True)
        rstd = aten.rsqrt.default(aten.add.Tensor(var, EPS))
        norm = aten.mul.Tensor(aten.sub.Tensor(arg0_1, mean), rstd)
        affine = aten.add.Tensor(aten.mul.Tensor(norm, _per_channel(arg3_1)), _per_channel(arg4_1))
        t = _upcast(_down(affine, arg0_1.dtype))
        silu = aten.div.Tensor(t, aten.add.Tensor(aten.exp.default(aten.neg.default(t)), 1))
        out = aten.constant_pad_nd.default(_down(silu, arg0_1.dtype), [0, 1, 0, 1], 0.0)
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
