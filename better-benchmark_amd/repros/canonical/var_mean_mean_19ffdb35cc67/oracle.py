"""
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
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

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
