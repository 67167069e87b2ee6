"""
MI355X oracle for mean_rmsnorm: y = x * rsqrt(mean(x^2) + eps) * gamma, rstd.

Kernel: hipo_rmsnorm_bf16 -- the row in registers (4 waves per row at
C = 4096), fp32 sum of squares reduced with DPP and a fixed-order LDS
combine, one rounding to bf16.  Algorithmic
bytes: 4 R C + 2 C + 4 R.
Replaces the Triton body of the reference's
repros/canonical/mean_4462ce967d63/oracle.py:65.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-05  # the graph constant of repro.py


@oracle_impl(hardware="MI355X", point="0390a437", description="RMSNorm, rows in registers")
@oracle_impl(hardware="MI355X", description="RMSNorm, shape-general")
def oracle_forward(inputs):
    x, gamma = inputs
    return hip_oracles.rmsnorm(x, gamma, EPS)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
