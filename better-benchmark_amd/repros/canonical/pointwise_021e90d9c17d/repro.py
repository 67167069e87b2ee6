"""
Canonical repro of the reference family pointwise_021e90d9c17d (timm
visformer_small, inference and training): attention output [B, heads, N, D]
back to an image [B, heads * D, H, W] -- swap the last two dims, make the
result contiguous, view it as NCHW.
Semantics of the reference's repros/canonical/pointwise_021e90d9c17d/repro.py:26-28
(permute [0, 1, 3, 2], clone in contiguous format, view); the two shape
points, with their model occurrence counts, are that dir's shapes.json.
A pure data movement: the result is bit-exact.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[128, 6, 49, 128]", _shape_param_0):
        swapped = torch.ops.aten.permute.default(arg0_1, [0, 1, 3, 2])
        dense = torch.ops.aten.clone.default(swapped, memory_format=torch.contiguous_format)
        return torch.ops.aten.view.default(dense, _shape_param_0)


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
