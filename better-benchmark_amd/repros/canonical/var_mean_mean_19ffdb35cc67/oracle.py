"""Gap diagnosis (classification: COOPERATIVE_SPLIT_K): this oracle computes the NCHW bf16 BatchNorm-training statistics as per-slice (mean, M2) partials over four-image slices (many workgroups per channel) merged in fp64, then normalises, applies ReLU and takes each plane's spatial mean in one epilogue pass with the plane in registers, whereas Inductor emits triton_red_fused_add_convert_element_type_copy__mul_rsqrt_squeeze_var_mean_0, one program per channel looping over all 128 images' 49-element planes (1024 programs for the whole reduction), then a persistent normalise + ReLU + mean kernel; Inductor cannot do this today because it does not split a per-channel reduction over the batch across workgroups when the channel count alone gives too few programs to fill the GPU; the fix is COOPERATIVE_SPLIT_K: split the channel reduction over batch slices with a deterministic merge.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
5b9efb9c, oracle 23.76 us, Inductor 29.8 us (ratio 1.254, GOOD); over the dir's 1
registered points: 1 GOOD.

MI355X oracle for var_mean_mean_19ffdb35cc67: BatchNorm training forward of
an NCHW bf16 activation (fp32 statistics, eps 1e-5) + ReLU + mean over H, W;
running statistics updated in place.

Kernel: hipo_batchnorm_nchw_act_mean_bf16 -- three launches: per (4 images,
64 channels) workgroup the slabs are staged through LDS with 16-byte loads
and each lane takes exact two-pass statistics of its channel's 7x7 segment;
a per-channel fp64 Chan merge in a fixed order (save_mean, save_rstd,
running statistics); the normalise + ReLU + spatial-mean pass over the same
slabs.  Algorithmic bytes: 2 N C H W (read) + 2 N C (write) + O(C).
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
