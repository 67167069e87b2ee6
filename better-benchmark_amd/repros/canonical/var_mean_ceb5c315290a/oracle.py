"""Gap diagnosis (classification: COOPERATIVE_SPLIT_K): this oracle computes the channels-last bf16 BatchNorm-training statistics as deterministic per-slice (mean, M2) partials merged in fp64, then writes the SiLU of the normalised value straight into the padded output in one epilogue pass, with the running statistics and saved statistics from the merge, whereas Inductor emits five kernels -- two levels of Welford split reduction, a finalize kernel, a pointwise affine kernel, and triton_poi_fused_add_constant_pad_nd_convert_element_type_div_exp_neg_4, a separate SiLU + pad kernel that reads the affine result back; Inductor cannot do this today because its BatchNorm-training lowering has no split-channel-statistics template whose epilogue produces the padded activation, so the activation and the pad cost an extra write and read of the whole tensor; the fix is COOPERATIVE_SPLIT_K: a split channel-statistics schedule feeding one epilogue that normalises, applies SiLU and writes the padded output.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
8026229d, oracle 163.82 us, Inductor 429.35 us (ratio 2.621, GOOD); over the dir's 2
registered points: 2 GOOD.

MI355X oracle for var_mean_ceb5c315290a: BatchNorm training forward of a
channels-last bf16 activation (fp32 statistics, eps 1e-3) + SiLU + a zero pad
of the bottom/right border; running statistics updated in place.

Kernel: hipo_batchnorm_nhwc_act_pad_bf16 -- three launches: per-slice
channel statistics (each workgroup instruction reads whole contiguous rows),
a per-channel fp64 Chan merge in a fixed order (save_mean, save_rstd, running
statistics), and the normalise + SiLU pass that writes the padded
channels-last output with 16-byte stores.  Algorithmic bytes: 2 N H W C
(read) + 2 N (H+1)(W+1) C (write) + O(C).
Replaces the Triton body of the reference's
repros/canonical/var_mean_ceb5c315290a/oracle.py:238.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-3  # graph constants of repro.py
MOMENTUM = 0.1
VAR_SCALE = 1.00000996502277


@oracle_impl(hardware="MI355X", point="cdca2f80", description="BN train + SiLU + pad, channels-last")
@oracle_impl(hardware="MI355X", point="8026229d", description="BN train + SiLU + pad, channels-last")
@oracle_impl(hardware="MI355X", description="BN train + SiLU + pad, channels-last, shape-general")
def oracle_forward(inputs):
    x, running_mean, running_var, gamma, beta = inputs
    mean, rstd, out = hip_oracles.batchnorm_nhwc_act_pad(
        x, gamma, beta, running_mean, running_var, momentum=MOMENTUM, eps=EPS,
        var_scale=VAR_SCALE, act="silu", pad_bottom=1, pad_right=1)
    return (mean, rstd, out, running_mean, running_var)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
