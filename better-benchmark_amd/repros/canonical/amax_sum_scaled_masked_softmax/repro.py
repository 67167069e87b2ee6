"""
Canonical repro: scaled, additively masked softmax over the last dim.
scores bf16 [384, 1024, 1024] ~ N(0, 1), scale 0.125,
mask bf16 [1024, 1024] (0 on/below the diagonal, -inf above) ->
out bf16 = softmax(scores * 0.125 + mask, -1), fp32 max/sum inside.
Pattern family of the reference's repros/canonical/amax_sum_192a3a5bd7ff
(scale, mask, fp32 amax/exp/sum/div; repro.py:23-44 there) and
amax_sum_20ccc18dda60 (bf16 broadcast additive bias + softmax).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
SCALE = 0.125


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[384, 1024, 1024]", arg1_1: "bf16[1024, 1024]"):
        mul: "bf16[384, 1024, 1024]" = torch.ops.aten.mul.Tensor(arg0_1, SCALE)
        add: "bf16[384, 1024, 1024]" = torch.ops.aten.add.Tensor(mul, arg1_1)
        softmax: "bf16[384, 1024, 1024]" = torch.ops.aten._softmax.default(add, -1, False)
        return softmax


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
