"""
Canonical repro of the reference family pointwise_8bb40810003c (timm / HF
training: an fp32 weight cast to bf16 and returned as its transpose and
itself).
Semantics of the reference's repros/canonical/pointwise_8bb40810003c/repro.py:24-29:
w [R, C] fp32 -> bf16, returned as (w.t(), w.t().t()): two views of one
contiguous bf16 tensor.  The shape points are that dir's shapes.json
points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "f32[1000, 2048]"):
        w = torch.ops.prims.convert_element_type.default(arg0_1, torch.bfloat16)
        wt = torch.ops.aten.permute.default(w, [1, 0])
        return (wt, torch.ops.aten.permute.default(wt, [1, 0]))


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
