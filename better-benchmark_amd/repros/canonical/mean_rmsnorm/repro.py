"""
Canonical repro: RMSNorm forward with fp32 statistics.
BASELINE config 4b: x bf16 [16384, 4096] ~ N(0, 1); gamma bf16 [4096] ~
N(1, 0.1); eps 1e-5 -> y bf16 [16384, 4096], rstd fp32 [16384].
y equals torch.nn.functional.rms_norm(x, [C], gamma, eps) (fp32 arithmetic,
one rounding to bf16), decomposed so rstd can be returned too.  Pattern
family of the reference's repros/canonical/mean_4462ce967d63/repro.py:23-38
(pow(2).mean(-1), + eps, rsqrt, scale).

Casts are "at least fp32" / "back to the input dtype" so the fp64 gate copy
computes in fp64.
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
    def forward(self, arg0_1: "bf16[16384, 4096]", arg1_1: "bf16[4096]"):
        convert_element_type: "f32[16384, 4096]" = _upcast(arg0_1)
        pow_1: "f32[16384, 4096]" = torch.ops.aten.pow.Tensor_Scalar(convert_element_type, 2)
        mean: "f32[16384, 1]" = torch.ops.aten.mean.dim(pow_1, [-1], True)
        add: "f32[16384, 1]" = torch.ops.aten.add.Tensor(mean, EPS)
        rsqrt: "f32[16384, 1]" = torch.ops.aten.rsqrt.default(add)
        mul: "f32[16384, 4096]" = torch.ops.aten.mul.Tensor(convert_element_type, rsqrt)
        mul_1: "f32[16384, 4096]" = torch.ops.aten.mul.Tensor(mul, _upcast(arg1_1))
        convert_element_type_1: "bf16[16384, 4096]" = \
            torch.ops.prims.convert_element_type.default(mul_1, arg0_1.dtype)
        squeeze: "f32[16384]" = torch.ops.aten.squeeze.dim(rsqrt, -1)
        return (convert_element_type_1, squeeze)


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
