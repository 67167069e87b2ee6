"""
MI355X oracle for pointwise_021e90d9c17d: [B, heads, N, D] -> contiguous
[B, heads, D, N], viewed as the NCHW image.

Kernel: hipo_transpose_last2 -- whole [N, D] matrices through LDS, one
workgroup per matrix: the input run read and the output run written as flat
streams of 16-byte non-temporal accesses, the element permutation done in
LDS (N = 49 and 196, so output rows are not 16-byte multiples).  Bit-exact.
Algorithmic bytes: 2 x numel x 2.
Replaces the Triton body of the reference's
repros/canonical/pointwise_021e90d9c17d/oracle.py:55-80
(_visformer_attention_to_image_kernel, :23).
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", point="6f902f84", description="last-two-dims transpose via LDS")
@oracle_impl(hardware="MI355X", point="918a77e3", description="last-two-dims transpose via LDS")
@oracle_impl(hardware="MI355X", description="last-two-dims transpose, shape-general")
def oracle_forward(inputs):
    x, out_shape = inputs
    return hip_oracles.transpose_last2(x).view(out_shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
