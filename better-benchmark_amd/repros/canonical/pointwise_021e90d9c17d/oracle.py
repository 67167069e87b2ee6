"""Gap diagnosis (classification: NEW_PATTERN): this oracle moves each small [N, D] matrix (N = 49 or 196) through LDS in one workgroup, so the input run is read and the output run written as flat streams of 16-byte non-temporal accesses with the permutation done in LDS, whereas Inductor emits triton_poi_fused_clone_permute_0, a Grid2D tiled transpose whose tiles cut across the 49- and 196-element rows, so its loads and stores are partial-width and masked; Inductor cannot do this today because its tiling picks YBLOCK x XBLOCK tiles over the logical axes and has no whole-matrix-per-workgroup path for matrices that fit in LDS; the fix is NEW_PATTERN: a small-matrix transpose template that streams whole matrices through LDS.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
918a77e3, oracle 16.48 us, Inductor 17.56 us (ratio 1.066, GOOD); over the dir's 2
registered points: 2 GOOD.

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
import hip_oracles
from oracle_harness import oracle_impl, oracle_main


@oracle_impl(hardware="MI355X", point="6f902f84", description="last-two-dims transpose via LDS")
@oracle_impl(hardware="MI355X", point="918a77e3", description="last-two-dims transpose via LDS")
@oracle_impl(hardware="MI355X", description="last-two-dims transpose, shape-general")
def oracle_forward(inputs):
    x, out_shape = inputs
    return hip_oracles.transpose_last2(x).view(out_shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
