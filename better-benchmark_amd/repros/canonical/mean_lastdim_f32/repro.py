"""
Canonical repro: fp32 row mean over the last dim.
x f32 [8192, 4096] ~ N(0, 1) -> out f32 [8192].
Pattern family of the reference's repros/canonical/mean_c9e1a8113328
(aten.mean.dim over the reduced axis, repro.py:26 there).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
# Input shapes/dtypes/generators live in the sibling shapes.json; the first
# point is the default.


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "f32[8192, 4096]"):
        mean: "f32[8192]" = torch.ops.aten.mean.dim(arg0_1, [-1])
        return mean


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
