"""
MI355X oracle for pointwise_9595e73ff43b: BatchNorm inference affine, ReLU6.

Kernel: hipo_bn_infer_act_bf16 (hip_oracles.bn_infer_act) in storage order:
channels-last with C % 8 == 0 keeps an 8-channel group's parameters in
registers per thread; NCHW stages the parameters of the channels a
workgroup touches in LDS.  16-byte non-temporal loads and stores.
Algorithmic bytes: 2 per element per bf16 input + 2 written (parameters
negligible).
Replaces the Triton body of the reference's
repros/canonical/pointwise_9595e73ff43b/oracle.py:107-127.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="ReLU6, shape-general")
def oracle_forward(inputs):
    mean, x, var, weight, bias = inputs
    return hip_oracles.bn_infer_act(x, mean, var, weight, bias, eps=1e-05, act="relu6")


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "8a10670c",
    "82cef4c9",
    "2cf7960f",
    "54640677",
    "1ee4ce98",
    "ba8126d9",
    "ebe204a7",
    "51719261",
    "d53a7e50",
    "2e1844e5",
    "9c97edfa",
    "3bdac97c",
    "66878456",
    "0598891b",
    "91334d30",
    "e5f12ec5",
    "94494857",
    "1cc752a4",
    "92d91bac",
    "3de61eda",
    "8dd8c35d",
    "522f10e2",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="ReLU6")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
