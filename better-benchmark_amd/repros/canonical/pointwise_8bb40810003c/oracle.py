"""
MI355X oracle for pointwise_8bb40810003c: an fp32 [R, C] tensor cast to
bf16 once, returned as its transpose view and itself (both views of the one
contiguous result, as eager returns them).

Kernel: hipo_cast_f32_to_bf16 over the contiguous input (storage order).
Algorithmic bytes: 4 + 2 per element.
Replaces the Triton body of the reference's
repros/canonical/pointwise_8bb40810003c/oracle.py:102-119.
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", description="fp32 -> bf16 cast, two views, shape-general")
def oracle_forward(inputs):
    (x,) = inputs
    w = hip_oracles.cast_storage(x.contiguous(), torch.bfloat16)
    return (w.permute(1, 0), w)


# one shapes.json point per distinct input shape (registrations are keyed by
# shape; points that differ only in strides share one); the kernel is
# shape-general
_POINTS = (
    "0cf39344",
    "ce1e0a23",
    "ae9f1068",
    "44a2434c",
    "f5f85987",
    "e24f40e4",
    "9e822d8f",
    "2e98be1c",
    "5cffd879",
    "e1aec24f",
    "aafa641b",
    "2613646b",
    "d29f2cfb",
    "5617a165",
    "ac612a70",
    "f0eaed89",
    "0a486f34",
    "ebcabf6d",
    "debf1fc5",
    "b30c1d04",
    "6c896102",
    "18173249",
    "62980a68",
    "af8b80d5",
    "9f2d4100",
    "1b40fbb6",
    "557311da",
    "5c0408c4",
    "b1ca53d6",
    "a1cb3860",
    "52d3c6a7",
    "01baa4eb",
    "43065864",
    "16e5c8c0",
    "fdcbaff1",
    "25dff7ef",
    "7cfcfe39",
    "19d8a989",
    "17dcd71b",
    "c4cfc269",
    "fb817d2a",
    "2d6d0114",
    "32e09daf",
    "e340bbdf",
    "1185642c",
    "d84d33a1",
    "af634b6e",
    "46c132a4",
    "8cf9b83f",
    "16d2cbc0",
    "62c6abfb",
    "595a24d8",
    "ec623101",
    "dc3e8b06",
    "040e49cd",
    "3798a6aa",
    "8aa63c17",
    "3851a1ae",
    "945f2c72",
    "6747b18a",
    "e692d575",
    "688f3d95",
    "559a6c52",
    "68efa070",
    "1c987e3e",
    "e583d54f",
    "2d7cdfa7",
    "e56e2d8f",
    "b016ff56",
    "2bb61127",
    "7a086584",
    "fdf8e815",
    "76ad9430",
    "b3e78a1b",
    "4f207a72",
    "58e39a16",
    "f4e93827",
    "60ceae96",
    "8d573313",
    "aa459734",
    "a7aca999",
    "a876c3bb",
    "afe477f0",
    "7b445016",
)
for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="fp32 -> bf16 cast, two views")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
