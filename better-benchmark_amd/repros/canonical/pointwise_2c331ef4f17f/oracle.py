"""
MI355X oracle for pointwise_2c331ef4f17f: BatchNorm inference affine, two affines added + ReLU.

Kernel: hipo_bn_infer_act_bf16 (hip_oracles.bn_infer_act) in storage order:
channels-last with C % 8 == 0 keeps an 8-channel group's parameters in
registers per thread; NCHW stages the parameters of the channels a
workgroup touches in LDS.  16-byte non-temporal loads and stores.
Algorithmic bytes: 2 per element per bf16 input + 2 written (parameters
negligible).
Replaces the Triton body of the reference's
repros/canonical/pointwise_2c331ef4f17f/oracle.py:305-306.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="two affines added + ReLU, shape-general")
def oracle_forward(inputs):
    mean, x, var, weight, bias, mean2, x2, var2, weight2, bias2 = inputs
    return hip_oracles.bn_infer_act(x, mean, var, weight, bias, eps=1e-05, act="relu", second=(x2, mean2, var2, weight2, bias2))


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "82978638",
    "3f9335c1",
    "b691104d",
    "7ee473b0",
    "f5c6beac",
    "d58c5fd0",
    "5c9d3965",
    "2c26d0d1",
    "e4b64a12",
    "1fa31355",
    "5e705d74",
    "88658619",
    "cf13ba44",
    "27f9b106",
    "cc596ad9",
    "68f48f4e",
    "eceeb412",
    "76020c9d",
    "0f0aebfd",
    "e006e72d",
    "83969398",
    "b188d91d",
    "795eaade",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="two affines added + ReLU")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
