"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle reduces a channels-last image over its H * W positions with every workgroup instruction reading whole contiguous position rows (all channels), fp32 sums per 8-channel group per thread and a fixed-order LDS merge, whereas Inductor emits triton_red_fused_mean_0, a looped reduction with one output per (image, channel) that walks the positions with channel-strided evict_first loads; Inductor cannot do this today because its reduction codegen keeps the reduced axis as the loop axis and does not re-tile a non-innermost reduction so that loads run along the contiguous channel axis; the fix is BANDWIDTH_BOUND: a column-reduction template for channels-last spatial means.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
2150fa2c, oracle 61.63 us, Inductor 65.11 us (ratio 1.056, GOOD); over the dir's 16
registered points: 10 AT_FLOOR, 6 GOOD.

MI355X oracle for mean_c9e1a8113328: spatial mean of a channels-last bf16
tensor over H, W (keepdim).

Kernel: hipo_spatial_mean_nhwc_bf16 -- per image a column reduction of the
[H*W, C] block: each workgroup instruction reads whole contiguous rows, every
thread keeps fp32 sums for one 8-channel group, partial sums meet in LDS in a
fixed order (and, when positions are split for parallelism, a second pass
adds the slices in order); images of at most 224 positions take one wave per
(image, 64-channel block) with every position in flight at once and an
xor-shuffle combine (no LDS).  Algorithmic bytes: 2 N H W C + 2 N C.
Replaces the Triton body of the reference's
repros/canonical/mean_c9e1a8113328/oracle.py:95 (_spatial_mean_cl_kernel, :11).
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

_POINTS = ("69db7514", "280fa7d2", "2645a53e", "4ca56f88", "d1686c77", "333b11d0",
           "547c8164", "f0a667e3", "44f1e75f", "4784273d", "3cf84b69", "2150fa2c",
           "6b68d184", "d3381898", "473b7062", "630d0797")


def oracle_forward(inputs):
    (x,) = inputs
    return hip_oracles.spatial_mean_nhwc(x, keepdim=True)


for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="channels-last spatial mean")(oracle_forward)
oracle_forward = oracle_impl(hardware="MI355X",
                             description="channels-last spatial mean, shape-general")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
