"""
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
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

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
