"""Gap diagnosis (classification: SCHEDULER_FUSION): this oracle keeps all N x H x W values of four channels in one workgroup's registers (staged through LDS with 8-byte loads, four waves per channel) and computes the channel statistics, the running statistics and the ReLU spatial means from them in one launch, reading x once, whereas Inductor emits triton_red_fused_add_convert_element_type_copy__mul_rsqrt_squeeze_var_mean_0, one program per channel looping over all 128 images' 49-element planes, then a persistent normalise + ReLU + mean kernel that reads x again; Inductor cannot do this today because its scheduler does not fuse a reduction with a consumer that needs the finished reduction over the same values unless the reduced values are one program's contiguous persistent block, and a channel's values here are N separate planes; the fix is SCHEDULER_FUSION: a persistent per-channel schedule that holds the channel's N x H x W values and runs the statistics and the epilogue on them in one kernel.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
5b9efb9c, oracle 19.76 us, Inductor 26.68 us (ratio 1.35, GOOD); over the dir's 1
registered points: 1 GOOD.

MI355X oracle for var_mean_mean_19ffdb35cc67: BatchNorm training forward of
an NCHW bf16 activation (fp32 statistics, eps 1e-5) + ReLU + mean over H, W;
running statistics updated in place.

Kernel: hipo_batchnorm_nchw_act_mean_bf16 -- at this point one launch: a
16-wave workgroup stages four channels' N x 7 x 7 values in LDS with 8-byte
loads, four waves per channel hold them in registers, take the channel
statistics in one pass about a value of the channel (fp32 per lane and wave,
fp64 over the waves, a fixed order), write save_mean, save_rstd and the
running statistics, and store the ReLU spatial means of every (image,
channel) -- x read once, no workspace.  Shapes whose channels do not fit a
workgroup take per-slice statistics, a per-channel fp64 merge and an
epilogue pass over the same slabs.  Algorithmic bytes: 2 N C H W (read) +
2 N C (write) + O(C).
Replaces the Triton body of the reference's
repros/canonical/var_mean_mean_19ffdb35cc67/oracle.py:167.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-05  # graph constants of repro.py
MOMENTUM = 0.1
VAR_SCALE = 1.0001594642002871


@oracle_impl(hardware="MI355X", point="5b9efb9c", description="BN train + ReLU + spatial mean, NCHW")
@oracle_impl(hardware="MI355X", description="BN train + ReLU + spatial mean, NCHW, shape-general")
def oracle_forward(inputs):
    x, running_mean, running_var, gamma, beta = inputs
    mean, rstd, out = hip_oracles.batchnorm_nchw_act_mean(
        x, gamma, beta, running_mean, running_var, momentum=MOMENTUM, eps=EPS,
        var_scale=VAR_SCALE, act="relu")
    return (mean, rstd, out, running_mean, running_var)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
