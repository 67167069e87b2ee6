"""
Canonical repro: per-channel bias + GELU(tanh), written channels-last.
x bf16 NCHW [128, 256, 56, 56] ~ N(0, 1), bias bf16 [256]
~ N(0, 0.1) -> out bf16 [128, 256, 56, 56] with channels-last strides.
Fuses the reference's tanh-GELU pattern
(repros/canonical/pointwise_2d969ac9ad59/repro.py:23-36) with its
permute + clone pattern (repros/canonical/pointwise_021e90d9c17d/repro.py:26-28).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[128, 256, 56, 56]", arg1_1: "bf16[256]"):
        view: "bf16[1, 256, 1, 1]" = torch.ops.aten.view.default(arg1_1, [1, -1, 1, 1])
        add: "bf16[128, 256, 56, 56]" = torch.ops.aten.add.Tensor(arg0_1, view)
        gelu: "bf16[128, 256, 56, 56]" = torch.ops.aten.gelu.default(add, approximate="tanh")
        clone: "bf16[128, 256, 56, 56]" = torch.ops.aten.clone.default(
            gelu, memory_format=torch.channels_last)
        return clone


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
