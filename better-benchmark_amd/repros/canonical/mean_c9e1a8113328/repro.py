"""
Canonical repro of the reference family mean_c9e1a8113328 (timm dm_nfnet_f0 /
nfnet_l0, inference and training): the spatial mean of a channels-last
bf16 activation, keepdim -- a reduction over the non-innermost axes H, W.
Semantics of the reference's repros/canonical/mean_c9e1a8113328/repro.py:23-27
(aten.mean.dim over [2, 3], keepdim); the 16 shape points, with their model
occurrence counts, are those of that dir's shapes.json.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[128, 1536, 8, 8]"):
        mean: "bf16[128, 1536, 1, 1]" = torch.ops.aten.mean.dim(arg0_1, [2, 3], True)
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
