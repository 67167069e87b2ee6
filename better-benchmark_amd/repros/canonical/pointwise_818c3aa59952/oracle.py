"""
MI355X oracle for pointwise_818c3aa59952: BatchNorm inference affine, no activation.

Kernel: hipo_bn_infer_act_bf16 (hip_oracles.bn_infer_act) in storage order:
channels-last with C % 8 == 0 keeps an 8-channel group's parameters in
registers per thread; NCHW stages the parameters of the channels a
workgroup touches in LDS.  16-byte non-temporal loads and stores.
Algorithmic bytes: 2 per element per bf16 input + 2 written (parameters
negligible).
Replaces the Triton body of the reference's
repros/canonical/pointwise_818c3aa59952/oracle.py:106-138.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="no activation, shape-general")
def oracle_forward(inputs):
    mean, x, var, weight, bias = inputs
    return hip_oracles.bn_infer_act(x, mean, var, weight, bias, eps=1e-05, act="none")


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "c6312c18",
    "1a06d794",
    "e9bc5ee0",
    "701aa9ad",
    "5540c28a",
    "4c825568",
    "4280fd00",
    "654b8cd3",
    "a118ca10",
    "a047c97b",
    "76c62ba9",
    "0a96753f",
    "4c724370",
    "ef49f65d",
    "c68fd75d",
    "ecb9a0d7",
    "3ddafcba",
    "3350df9a",
    "e987d149",
    "1fca60d1",
    "8e74e392",
    "b72bb793",
    "def42dcc",
    "d6d99242",
    "9f949812",
    "6129a191",
    "5959a6c3",
    "bd03f6f7",
    "6349ba76",
    "e2542415",
    "d132f392",
    "4552b8d5",
    "40a7d00c",
    "5e9ad3e0",
    "4f4eacf9",
    "7395f576",
    "908bdc99",
    "d5e26824",
    "05028dd8",
    "261d5bdd",
    "aaa0fce0",
    "ced04216",
    "d773a707",
    "d820ae29",
    "fa15eadf",
    "6e30cacc",
    "017f27d2",
    "5c1756a4",
    "13e72620",
    "f3036c42",
    "9a05b224",
    "0ba75884",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="no activation")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
