"""
Canonical repro of the reference family pointwise_2d969ac9ad59 (HF Albert,
DistillGPT2, GPT-2, GPT-J, GPT-Neo, FNet; inference and training): the
decomposed tanh GELU of a transformer MLP activation, between two views.
Semantics of the reference's repros/canonical/pointwise_2d969ac9ad59/repro.py:23-36:
0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3))) as eight eager ops,
each rounding to the input dtype (bf16 at five points, fp32 at one); the
six shape points, with their model occurrence counts, are that dir's
shapes.json.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[4096, 16384]", _shape_param_0, _shape_param_1):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        half = torch.ops.aten.mul.Tensor(view, 0.5)
        cube = torch.ops.aten.pow.Tensor_Scalar(view, 3.0)
        inner = torch.ops.aten.add.Tensor(view, torch.ops.aten.mul.Tensor(cube, 0.044715))
        th = torch.ops.aten.tanh.default(torch.ops.aten.mul.Tensor(inner, 0.7978845608028654))
        out = torch.ops.aten.mul.Tensor(half, torch.ops.aten.add.Tensor(th, 1.0))
        return torch.ops.aten.view.default(out, _shape_param_1)


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
