"""
Canonical repro of the reference family pointwise_e6ddc8e897ec (timm inference: BN + residual add).
Semantics of the reference's repros/canonical/pointwise_e6ddc8e897ec/repro.py:24-46:
BatchNorm inference in eager's ops -- per channel
reciprocal(sqrt(f32(var) + 1e-05)) * 1, per element
bf16(((x - mean) * inv) * weight + bias) in fp32 -- then a bf16 residual add.  bf16
parameters [C], bf16 [N, C, H, W] activations, contiguous or channels-last
as each shapes.json point gives.  The shape points are that dir's
shapes.json points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[384]", arg1_1: "bf16[128, 384, 8, 8]", arg2_1: "bf16[384]", arg3_1: "bf16[384]", arg4_1: "bf16[384]", arg5_1: "bf16[128, 384, 8, 8]"):
        def affine(x, mean, var, w, b):
            m = torch.ops.aten.unsqueeze.default(torch.ops.aten.unsqueeze.default(
                torch.ops.prims.convert_element_type.default(mean, torch.float32), -1), -1)
            sub = torch.ops.aten.sub.Tensor(x, m)
            v = torch.ops.prims.convert_element_type.default(var, torch.float32)
            inv = torch.ops.aten.mul.Tensor(torch.ops.aten.reciprocal.default(
                torch.ops.aten.sqrt.default(torch.ops.aten.add.Tensor(v, 1e-05))), 1)
            inv = torch.ops.aten.unsqueeze.default(torch.ops.aten.unsqueeze.default(inv, -1), -1)
            mul_1 = torch.ops.aten.mul.Tensor(sub, inv)
            wu = torch.ops.aten.unsqueeze.default(torch.ops.aten.unsqueeze.default(w, -1), -1)
            bu = torch.ops.aten.unsqueeze.default(torch.ops.aten.unsqueeze.default(b, -1), -1)
            add_1 = torch.ops.aten.add.Tensor(torch.ops.aten.mul.Tensor(mul_1, wu), bu)
            return torch.ops.prims.convert_element_type.default(add_1, torch.bfloat16)
        return torch.ops.aten.add.Tensor(affine(arg1_1, arg0_1, arg2_1, arg3_1, arg4_1), arg5_1)


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
