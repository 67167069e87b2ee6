"""
Canonical repro of the reference family amax_sum_20ccc18dda60 (HF TrOCR
inference): attention softmax with an additive bias broadcast over heads.
Semantics of the reference's repros/canonical/amax_sum_20ccc18dda60/repro.py:23-35:
scores [1024, 256, 256] viewed [64, 16, 256, 256] + bias [64, 1, 256, 256]
(bf16 add), then fp32 amax / exp / sum / div, bf16 out; the shape point is
that dir's shapes.json point.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


def _upcast(t):
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[1024, 256, 256]", arg1_1: "bf16[64, 1, 256, 256]",
                _shape_param_0, _shape_param_1):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        add = torch.ops.aten.add.Tensor(view, arg1_1)
        s = _upcast(torch.ops.aten.view.default(add, _shape_param_1))
        amax = torch.ops.aten.amax.default(s, [-1], True)
        e = torch.ops.aten.exp.default(torch.ops.aten.sub.Tensor(s, amax))
        total = torch.ops.aten.sum.dim_IntList(e, [-1], True)
        return torch.ops.prims.convert_element_type.default(
            torch.ops.aten.div.Tensor(e, total), arg0_1.dtype)


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
