"""
Canonical repro of the reference family pointwise_ccd411f2a45d (timm / HF:
fp32 weights and activations cast to bf16).
Semantics of the reference's repros/canonical/pointwise_ccd411f2a45d/repro.py:24-27:
one convert_element_type fp32 -> bf16 (round to nearest even) that keeps
the input's strides.  The shape points are that dir's shapes.json
points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "f32[1000]"):
        return torch.ops.prims.convert_element_type.default(arg0_1, torch.bfloat16)


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
