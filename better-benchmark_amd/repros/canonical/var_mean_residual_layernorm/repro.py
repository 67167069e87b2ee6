"""
Canonical repro: residual add + LayerNorm forward with fp32 statistics.
BASELINE config 4a: x, residual bf16 [16384, 4096] ~ N(0, 1); gamma bf16
[4096] ~ N(1, 0.1); beta bf16 [4096] ~ N(0, 0.1); eps 1e-5 ->
h = x + residual (bf16), y = LayerNorm(h) (bf16), mean and rstd (fp32
[16384]).  Same graph as the reference's
repros/canonical/var_mean_80e7ff4dee7f/repro.py:23-39 (bf16 add, fp32
var_mean with correction 0, rsqrt, affine, bf16), with h, mean and rstd
also returned.  Statistics are taken over the bf16-rounded h.

Casts are written "at least fp32" / "back to the input dtype", so the fp64
copy used by the numerics gate (`Repro().double()` on fp64 inputs) computes
the whole graph in fp64.
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
    def forward(self, arg0_1: "bf16[16384, 4096]", arg1_1: "bf16[16384, 4096]",
                arg2_1: "bf16[4096]", arg3_1: "bf16[4096]"):
        add: "bf16[16384, 4096]" = torch.ops.aten.add.Tensor(arg0_1, arg1_1)
        convert_element_type: "f32[16384, 4096]" = _upcast(add)
        var_mean = torch.ops.aten.var_mean.correction(
            convert_element_type, [-1], correction=0, keepdim=True)
        getitem: "f32[16384, 1]" = var_mean[0]
        getitem_1: "f32[16384, 1]" = var_mean[1]
        sub: "f32[16384, 4096]" = torch.ops.aten.sub.Tensor(convert_element_type, getitem_1)
        add_1: "f32[16384, 1]" = torch.ops.aten.add.Tensor(getitem, EPS)
        rsqrt: "f32[16384, 1]" = torch.ops.aten.rsqrt.default(add_1)
        mul: "f32[16384, 4096]" = torch.ops.aten.mul.Tensor(sub, rsqrt)
        mul_1: "f32[16384, 4096]" = torch.ops.aten.mul.Tensor(mul, arg2_1)
        add_2: "f32[16384, 4096]" = torch.ops.aten.add.Tensor(mul_1, arg3_1)
        convert_element_type_1: "bf16[16384, 4096]" = \
            torch.ops.prims.convert_element_type.default(add_2, arg0_1.dtype)
        squeeze: "f32[16384]" = torch.ops.aten.squeeze.dim(getitem_1, -1)
        squeeze_1: "f32[16384]" = torch.ops.aten.squeeze.dim(rsqrt, -1)
        return (add, convert_element_type_1, squeeze, squeeze_1)


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
