"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes relu(x).mean over 169-element planes by having each wave read eight consecutive planes as one flat non-temporal stream of 16-byte loads, stage them in LDS and sum each plane over 8 lanes in a fixed order, whereas Inductor emits triton_per_fused_mean_relu_0, a persistent reduction with one 169-element plane per program row and masked scalar-width loads (a plane is not a multiple of 16 bytes); Inductor cannot do this today because its reduction layouts load each reduction row separately and cannot vectorise rows whose length breaks 16-byte alignment; the fix is BANDWIDTH_BOUND: a layout that streams several consecutive short rows as one vector stream and splits them in LDS.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
dad91233, oracle 13.56 us, Inductor 13.64 us (ratio 1.006, AT_FLOOR); over the dir's 1
registered points: 1 AT_FLOOR.

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
import hip_oracles
from oracle_harness import oracle_impl, oracle_main


@oracle_impl(hardware="MI355X", point="dad91233", description="ReLU + NCHW spatial mean")
@oracle_impl(hardware="MI355X", description="ReLU + NCHW spatial mean, shape-general")
def oracle_forward(inputs):
    x, out_shape = inputs
    n, c = x.shape[0], x.shape[1]
    return hip_oracles.row_mean_bf16(x.reshape(n * c, -1), relu=True).view(out_shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
