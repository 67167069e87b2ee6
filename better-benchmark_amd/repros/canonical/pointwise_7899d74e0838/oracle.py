"""
MI355X oracle for pointwise_7899d74e0838: BatchNorm inference affine, ReLU (eps 1e-3).

Kernel: hipo_bn_infer_act_bf16 (hip_oracles.bn_infer_act) in storage order:
channels-last with C % 8 == 0 keeps an 8-channel group's parameters in
registers per thread; NCHW stages the parameters of the channels a
workgroup touches in LDS.  16-byte non-temporal loads and stores.
Algorithmic bytes: 2 per element per bf16 input + 2 written (parameters
negligible).
Replaces the Triton body of the reference's
repros/canonical/pointwise_7899d74e0838/oracle.py:241-293.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="ReLU (eps 1e-3), shape-general")
def oracle_forward(inputs):
    mean, x, var, weight, bias = inputs
    return hip_oracles.bn_infer_act(x, mean, var, weight, bias, eps=0.001, act="relu")


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "aeef24a2",
    "d0015d69",
    "79f50b00",
    "45fcf39e",
    "6b130750",
    "466338df",
    "2eaf76ca",
    "5ecba4cf",
    "2869e39e",
    "8a535339",
    "f868ccff",
    "2b758769",
    "a034af1b",
    "4c825568",
    "3d7c0f11",
    "76836be5",
    "37cf4567",
    "09d7b0e3",
    "ff6665c7",
    "2d204c68",
    "0a96753f",
    "c7c6ed1f",
    "e7ac2695",
    "5ddd3fd5",
    "b88e53cc",
    "9c97edfa",
    "55c49b50",
    "9ffe1d7a",
    "d0456ef8",
    "dc068d28",
    "23b42229",
    "8273eec8",
    "fe78a763",
    "fb1609c3",
    "3a805d91",
    "f9b980a0",
    "9a46a7c3",
    "29619cda",
    "49317bb2",
    "15c8ba03",
    "5536024c",
    "706b5a8b",
    "0c615bbc",
    "86d8b817",
    "a01c3bbe",
    "ba61c626",
    "bc2770a8",
    "9e8f8bc2",
    "8004dcee",
    "6039b181",
    "d438d876",
    "b6537524",
    "cc855e4e",
    "27be3f93",
    "a3bf2c8d",
    "0fe88f70",
    "6558df98",
    "793856d7",
    "c2f1485a",
    "78e9098c",
    "4fbb328e",
    "c1f1985a",
    "b83c3106",
    "82781865",
    "3a0fa905",
    "e3b17b69",
    "d6d70882",
    "c9277843",
    "6cc76740",
    "08df9f87",
    "a952c87d",
    "51b8f364",
    "e78adaa5",
    "09db272d",
    "1f81c187",
    "b5cedc58",
    "c78ca241",
    "11ab0e65",
    "4194c732",
    "05028dd8",
    "4f218228",
    "0ce7c2f4",
    "535abe76",
    "3f17dc95",
    "d957323e",
    "7fd9f949",
    "2b7370d5",
    "6ff82f3b",
    "f50736b8",
    "ad2ff10f",
    "7ebdbaf5",
    "8380c440",
    "e3fcf83d",
    "20f76211",
    "2ff0039c",
    "93683cfe",
    "6b05bfa0",
    "6a1621d9",
    "f7d56653",
    "c7ca5fcc",
    "eff1e63e",
    "18ebcf69",
    "13e72620",
    "b30eafb6",
    "f3036c42",
    "eb73312d",
    "9a05b224",
    "c356b4b1",
    "a8109c98",
    "a9c4f100",
    "7e261bd0",
    "fe80f1ea",
    "217063c8",
    "13bff0d2",
    "23eaa07b",
    "dd92c2d0",
    "357d64ea",
    "e84dbb88",
    "839e83c4",
    "608e0114",
    "a2b8c17d",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="ReLU (eps 1e-3)")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
