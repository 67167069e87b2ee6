"""
Canonical repro of the reference family amax_sum_fa4cc85fe5ad (HF T5 / MT5
inference): the attention softmax with no bias or scale.
Semantics of the reference's repros/canonical/amax_sum_fa4cc85fe5ad/repro.py:24-36:
scores [B, Q, K] viewed [b, h, Q, K], fp32 amax / exp / sum / div over the
last dim, bf16 out, expanded and viewed back to [B, Q, K]; the shape points
are that dir's shapes.json points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3


def _upcast(t):
    # fp32 for bf16 scores (the graph's convert_element_type); an fp64 copy
    # of the module (the numerics gate's anchor) stays in fp64.
    return torch.ops.prims.convert_element_type.default(
        t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[192, 128, 128]", _shape_param_0, _shape_param_1,
                _shape_param_2):
        view = torch.ops.aten.view.default(arg0_1, _shape_param_0)
        s = _upcast(view)
        amax = torch.ops.aten.amax.default(s, [-1], True)
        e = torch.ops.aten.exp.default(torch.ops.aten.sub.Tensor(s, amax))
        total = torch.ops.aten.sum.dim_IntList(e, [-1], True)
        p = torch.ops.prims.convert_element_type.default(
            torch.ops.aten.div.Tensor(e, total), torch.bfloat16)
        expand = torch.ops.aten.expand.default(p, _shape_param_1)
        return torch.ops.aten.view.default(expand, _shape_param_2)


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
