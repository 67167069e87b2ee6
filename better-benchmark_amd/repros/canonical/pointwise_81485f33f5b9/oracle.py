"""
MI355X oracle for pointwise_81485f33f5b9: BatchNorm inference affine, residual add + ReLU.

Kernel: hipo_bn_infer_act_bf16 (hip_oracles.bn_infer_act) in storage order:
channels-last with C % 8 == 0 keeps an 8-channel group's parameters in
registers per thread; NCHW stages the parameters of the channels a
workgroup touches in LDS.  16-byte non-temporal loads and stores.
Algorithmic bytes: 2 per element per bf16 input + 2 written (parameters
negligible).
Replaces the Triton body of the reference's
repros/canonical/pointwise_81485f33f5b9/oracle.py:156-202.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="residual add + ReLU, shape-general")
def oracle_forward(inputs):
    mean, x, var, weight, bias, residual = inputs
    return hip_oracles.bn_infer_act(x, mean, var, weight, bias, eps=1e-05, act="relu", residual=residual)


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "85db042c",
    "0af2d571",
    "3aeeed95",
    "fd6e1886",
    "cd893d5b",
    "28e6bebb",
    "08581e62",
    "50714806",
    "4c0cf88f",
    "6b748dff",
    "7111f2e4",
    "2e6c4615",
    "e626f5a9",
    "40170966",
    "e2161da4",
    "72f4709b",
    "cce8fbb3",
    "2f5dac5e",
    "3bac8de4",
    "592ca691",
    "e20a55a6",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="residual add + ReLU")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
