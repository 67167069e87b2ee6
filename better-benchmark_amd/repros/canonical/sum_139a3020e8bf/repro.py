"""
Canonical repro of the reference family sum_139a3020e8bf (timm ViT / DeiT /
BEiT / SigLIP and HF BERT-style training): the gradient through an erf GELU
and its bias gradient.
Semantics of the reference's repros/canonical/sum_139a3020e8bf/repro.py:24-48:
grad and x [R, C] bf16 (viewed [B, T, C] and back), in fp32
  d = 0.5 (erf(x / sqrt 2) + 1) + x (exp(-x^2 / 2) / sqrt(2 pi)),
  y = bf16(grad * d) [R, C], returned with its transpose view [C, R], and
  colsum = f32(bf16(sum over R of y in fp32)) [C].
The shape points are that dir's shapes.json points.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
from repro_harness import benchmark_repro, make_inputs_from_config, load_shape_configs  # noqa: E402

_repro_version = 3

A = torch.ops.aten
P = torch.ops.prims


def _upcast(t):
    # fp32 for bf16 inputs (the graph's convert_element_type); an fp64 copy
    # of the module (the numerics gate's anchor) stays in fp64.
    return P.convert_element_type.default(t, torch.promote_types(t.dtype, torch.float32))


class Repro(torch.nn.Module):
    def forward(self, arg0_1: "bf16[25216, 3072]", arg1_1: "bf16[25216, 3072]",
                _shape_param_0, _shape_param_1, _shape_param_2, _shape_param_3):
        g = _upcast(A.view.default(arg0_1, _shape_param_0))
        x = _upcast(A.view.default(arg1_1, _shape_param_1))
        cdf = A.mul.Tensor(A.add.Tensor(A.erf.default(A.mul.Tensor(x, 0.7071067811865476)), 1), 0.5)
        e = A.exp.default(A.mul.Tensor(A.mul.Tensor(x, x), -0.5))
        pdf = A.mul.Tensor(x, A.mul.Tensor(e, 0.3989422804014327))
        y = P.convert_element_type.default(A.mul.Tensor(g, A.add.Tensor(cdf, pdf)),
                                           torch.bfloat16)
        y2 = A.view.default(y, _shape_param_2)
        yt = A.permute.default(y2, [1, 0])
        # the graph's fp32 sum (dtype=float32); fp64 in the gate's anchor copy
        s = A.sum.dim_IntList(y2, [0], True, dtype=g.dtype)
        colsum = P.convert_element_type.default(
            P.convert_element_type.default(A.view.default(s, _shape_param_3), torch.bfloat16),
            s.dtype)
        return (y2, yt, colsum)


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
