"""
Canonical repro: BatchNorm training forward + ReLU with running-stat update.
x f32 NCHW [128, 256, 56, 56] ~ N(0.5, 2); gamma ~
N(1, 0.1); beta ~ N(0, 0.1); running_mean = 0, running_var = 1 (f32 [256]);
momentum 0.1; eps 1e-5 -> y = relu(bn(x)), save_mean, save_invstd, and the
running statistics updated in place (unbiased variance).  Pattern family of
the reference's repros/canonical/var_mean_mean_19ffdb35cc67/repro.py:23-54
(var_mean over [0, 2, 3], running-stat copies) and
var_mean_ceb5c315290a/repro.py:27-39.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3
MOMENTUM = 0.1
EPS = 1e-05


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "f32[128, 256, 56, 56]", arg1_1: "f32[256]",
                arg2_1: "f32[256]", arg3_1: "f32[256]", arg4_1: "f32[256]"):
        native_batch_norm = torch.ops.aten.native_batch_norm.default(
            arg0_1, arg1_1, arg2_1, arg3_1, arg4_1, True, MOMENTUM, EPS)
        getitem: "f32[128, 256, 56, 56]" = native_batch_norm[0]
        getitem_1: "f32[256]" = native_batch_norm[1]
        getitem_2: "f32[256]" = native_batch_norm[2]
        relu: "f32[128, 256, 56, 56]" = torch.ops.aten.relu.default(getitem)
        return (relu, getitem_1, getitem_2, arg3_1, arg4_1)


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
