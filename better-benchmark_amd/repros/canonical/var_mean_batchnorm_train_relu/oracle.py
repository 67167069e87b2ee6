"""
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
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

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
