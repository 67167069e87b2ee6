"""
MI355X oracle for mean_b402ee209d0b: relu(x).mean([-1, -2]) of a contiguous
NCHW bf16 tensor, as [N, C].

Kernel: hipo_row_mean_bf16 (relu) over the N * C planes as rows of H * W
elements -- each wave reads 8 consecutive planes (a whole number of 16-byte
vectors whatever H * W is) as one flat non-temporal stream, stages them in
LDS, sums each plane in fp32 over 8 lanes in a fixed order and rounds the
mean to bf16 once; ReLU keeps NaN.  Algorithmic bytes: 2 N C H W + 2 N C.
Replaces the Triton body of the reference's
repros/canonical/mean_b402ee209d0b/oracle.py:53-80 (_relu_spatial_mean_kernel, :23).
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", point="dad91233", description="ReLU + NCHW spatial mean")
@oracle_impl(hardware="MI355X", description="ReLU + NCHW spatial mean, shape-general")
def oracle_forward(inputs):
    x, out_shape = inputs
    n, c = x.shape[0], x.shape[1]
    return hip_oracles.row_mean_bf16(x.reshape(n * c, -1), relu=True).view(out_shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
