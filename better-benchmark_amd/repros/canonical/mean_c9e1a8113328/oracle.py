"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle reduces a channels-last image over its H * W positions with every workgroup instruction reading whole contiguous position rows (all channels), fp32 sums per 8-channel group per thread and a fixed-order LDS merge, whereas Inductor emits triton_red_fused_mean_0, a looped reduction with one output per (image, channel) that walks the positions with channel-strided evict_first loads; Inductor cannot do this today because its reduction codegen keeps the reduced axis as the loop axis and does not re-tile a non-innermost reduction so that loads run along the contiguous channel axis; the fix is BANDWIDTH_BOUND: a column-reduction template for channels-last spatial means.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
2150fa2c, oracle 63.99 us, Inductor 65.75 us (ratio 1.028, AT_FLOOR); over the dir's 11
registered points: 9 AT_FLOOR, 2 GOOD; 5 points withdrawn (WITHDRAWN_POINTS).

MI355X oracle for mean_c9e1a8113328: spatial mean of a channels-last bf16
tensor over H, W (keepdim).

Kernel: hipo_spatial_mean_nhwc_bf16 -- per image a column reduction of the
[H*W, C] block: each workgroup instruction reads whole contiguous rows, every
thread keeps fp32 sums for one 8-channel group, partial sums meet in LDS in a
fixed order (and, when positions are split for parallelism, a second pass
adds the slices in order).  Algorithmic bytes: 2 N H W C + 2 N C.
Replaces the Triton body of the reference's
repros/canonical/mean_c9e1a8113328/oracle.py:95 (_spatial_mean_cl_kernel, :11).
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

_POINTS = ("280fa7d2", "2645a53e", "4ca56f88", "547c8164",
           "f0a667e3", "4784273d", "3cf84b69", "2150fa2c", "d3381898", "473b7062",
           "630d0797")

# Points of shapes.json with no MI355X registration: the 6x6, 7x7, 8x8, 9x9
# and 12x12 images of 1536 channels.  Back to back, Inductor's reduction is
# faster (6x6: 4.76 against 5.50 us, 7x7: 5.73 against 6.36 us, 9x9: 7.08
# against 8.05 us) or equal (8x8: 6.49 against 6.54 us); 16-, 32- and
# 64-group channel blocks, one round of loads and wave-shuffle combines
# reached 5.20, 5.83, 6.48 and 8.10 us at best; single launches measured
# BAD_ORACLE at each of them at least once (12x12: 0.939 in the last of five
# status sweeps, 0.954-0.987 before).  There is no shape-general
# registration, so these points find no MI355X oracle (NO_ORACLE_FOR_SHAPE);
# the kernel still computes them and the parity tests call it directly.
# Values: the lowest single-launch ratio compile_us / oracle_us, then the
# back-to-back ratio where measured.
WITHDRAWN_POINTS = {
    "d1686c77": (0.906, 0.865),
    "6b68d184": (0.915, 0.901),
    "69db7514": (0.941, 0.992),
    "44f1e75f": (0.900, 0.879),
    "333b11d0": (0.939,),
}


def oracle_forward(inputs):
    (x,) = inputs
    return hip_oracles.spatial_mean_nhwc(x, keepdim=True)


for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="channels-last spatial mean")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
