"""
MI355X oracle for pointwise_e6ddc8e897ec: BatchNorm inference affine, residual add.

Kernel: hipo_bn_infer_act_bf16 (hip_oracles.bn_infer_act) in storage order:
channels-last with C % 8 == 0 keeps an 8-channel group's parameters in
registers per thread; NCHW stages the parameters of the channels a
workgroup touches in LDS.  16-byte non-temporal loads and stores.
Algorithmic bytes: 2 per element per bf16 input + 2 written (parameters
negligible).
Replaces the Triton body of the reference's
repros/canonical/pointwise_e6ddc8e897ec/oracle.py:142-174.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="residual add, shape-general")
def oracle_forward(inputs):
    mean, x, var, weight, bias, residual = inputs
    return hip_oracles.bn_infer_act(x, mean, var, weight, bias, eps=1e-05, act="none", residual=residual)


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "1b9786b5",
    "cbfa3b6c",
    "dee7c6c7",
    "2cdd53e8",
    "02ba49e6",
    "059bf3db",
    "342a6237",
    "c8441aee",
    "fc6552ee",
    "50e4898b",
    "3bc177c9",
    "a2ab0ad0",
    "8858d870",
    "cbb247bc",
    "6f6fdd1f",
    "661bb0c6",
    "9147e0bf",
    "6834e84b",
    "4273c1f9",
    "127b8ac2",
    "0f6a0e52",
    "cce36204",
    "e62d3519",
    "7638df56",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="residual add")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
