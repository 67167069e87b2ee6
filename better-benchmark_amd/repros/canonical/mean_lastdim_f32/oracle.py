"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle reduces each 4096-wide fp32 row with eight waves that issue all of the row's non-temporal 16-byte loads at once (1 KiB per instruction) and combine in a fixed order (DPP within the wave, LDS across waves), whereas Inductor emits triton_red_fused_mean_0, a looped reduction that walks each row in R0_BLOCK chunks with evict_first cached loads from one program per row block; Inductor cannot do this today because its ROCm reduction heuristics neither split one row across several waves with the whole row in flight nor emit streaming (non-temporal) loads for an input read exactly once; the fix is BANDWIDTH_BOUND: a multi-wave row-reduction template with non-temporal loads for single-use inputs.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
b84ae979, oracle 29.88 us, Inductor 30.04 us (ratio 1.005, AT_FLOOR); over the dir's 3
registered points: 2 AT_FLOOR, 1 BAD_ORACLE.  That one, [7, 333] at 0.941, was the
scalar kernel issuing one load at a time; with eight loads per lane in flight the
same protocol measured 0.994 and 1.003 (12.92-13.04 us against 12.96), AT_FLOOR.

MI355X oracle for mean_lastdim_f32: x.mean(dim=-1) on fp32 [R, C].

Kernel: hipo_row_mean_f32 (libhip_oracles.so) -- up to 8 waves per row,
non-temporal 16-byte lane-interleaved loads (1 KiB per load instruction),
fp32 accumulation, DPP wave reduction, fixed-order LDS combine.  Algorithmic bytes: 4 R C + 4 R.
Replaces the Triton body of the reference's
repros/canonical/mean_c9e1a8113328/oracle.py:95 (row mode, :45).
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main


@oracle_impl(hardware="MI355X", point="b84ae979", description="row mean, waves per row")
@oracle_impl(hardware="MI355X", description="row mean, shape-general")
def oracle_forward(inputs):
    (x,) = inputs
    return hip_oracles.row_mean(x)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
