"""Gap diagnosis (classification: COOPERATIVE_SPLIT_K): this oracle reads x once: 256 persistent workgroups (one per CU) each hold a 196 KiB slab of one channel in registers, publish fp32 (count, mean, M2) triples, merge the eight slabs of a channel in fp64 after a bounded tagged-word exchange, and normalise + ReLU from registers while the next round's loads are in flight, whereas Inductor emits three kernels -- triton_red_fused__native_batch_norm_legit_functional_0 (a Welford split over four chunks per channel), a finalize kernel that also writes the running statistics, and triton_poi_fused__native_batch_norm_legit_functional_relu_2, which reads x a second time to normalise; Inductor cannot do this today because it has no cooperative (grid-synchronised) reduction template that keeps the reduced data resident for the epilogue, so a reduction over the non-innermost axes of NCHW x costs a second 411 MB read; the fix is COOPERATIVE_SPLIT_K: a single-read BatchNorm-training schedule with a cross-workgroup exchange of the channel statistics.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
ce16d05d, oracle 160.26 us, Inductor 206.42 us (ratio 1.288, GOOD); over the dir's 3
registered points: 2 AT_FLOOR, 1 GOOD.

MI355X oracle for var_mean_batchnorm_train_relu: BatchNorm training forward
+ ReLU, save_mean / save_invstd, running statistics updated in place.

Kernel: hipo_batchnorm_train_fwd_f32 -- one persistent launch that reads x
once: each workgroup holds its slab of a channel in registers, the slabs'
Welford partials are exchanged between workgroups (tagged atomic words) and
merged with Chan's formula in fp64, then the same registers are normalised
(affine + ReLU) and stored; running statistics use the unbiased variance.
Algorithmic bytes: 4 N C H W (read) + 4 N C H W (write) + O(C).
Replaces the Triton bodies of the reference's
repros/canonical/var_mean_mean_19ffdb35cc67/oracle.py:167 and
repros/canonical/var_mean_ceb5c315290a/oracle.py:238.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

MOMENTUM = 0.1  # graph constants of repro.py
EPS = 1e-05


@oracle_impl(hardware="MI355X", point="ce16d05d", description="BN train fwd + ReLU, single pass")
@oracle_impl(hardware="MI355X", description="BN train fwd + ReLU, shape-general")
def oracle_forward(inputs):
    x, gamma, beta, running_mean, running_var = inputs
    y, save_mean, save_invstd = hip_oracles.batchnorm_train(
        x, gamma, beta, running_mean, running_var, momentum=MOMENTUM, eps=EPS, relu=True)
    return (y, save_mean, save_invstd, running_mean, running_var)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
