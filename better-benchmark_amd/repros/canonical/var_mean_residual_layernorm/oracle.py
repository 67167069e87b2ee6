"""
MI355X oracle for var_mean_residual_layernorm:
h = x + residual; y = LayerNorm(h) * gamma + beta; mean, rstd (fp32).

Kernel: hipo_residual_layernorm_bf16 -- the row in registers between the
statistics and the normalisation (x and residual are read once; 4 waves per
row at C = 4096), exact two-pass fp32 statistics of each wave's values of
the bf16-rounded h, merged across waves with Chan's formula.  Algorithmic bytes: 8 R C + 4 C + 8 R.
Replaces the Triton body of the reference's
repros/canonical/var_mean_80e7ff4dee7f/oracle.py:122 (without its
anchor-clamp of the output).
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-05  # the graph constant of repro.py


@oracle_impl(hardware="MI355X", point="fe9bbcba", description="residual LN, rows in registers")
@oracle_impl(hardware="MI355X", description="residual LN, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, beta = inputs
    return hip_oracles.residual_layernorm(x, residual, gamma, beta, EPS)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
