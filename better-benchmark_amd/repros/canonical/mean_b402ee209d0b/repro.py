"""
Canonical repro of the reference family mean_b402ee209d0b (torchbench
squeezenet1_1, inference and training): the classifier head -- ReLU, then
the spatial mean of an NCHW bf16 map, viewed as [N, C].
Semantics of the reference's repros/canonical/mean_b402ee209d0b/repro.py:23-27
(relu, mean.dim over [-1, -2] keepdim, view); the shape point, with its
model occurrence count, is that dir's shapes.json.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[16, 1000, 13, 13]", _shape_param_0):
        act = torch.ops.aten.relu.default(arg0_1)
        pooled = torch.ops.aten.mean.dim(act, [-1, -2], True)
        return torch.ops.aten.view.default(pooled, _shape_param_0)


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
