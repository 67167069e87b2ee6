"""
MI355X oracle for var_mean_80e7ff4dee7f: residual add + LayerNorm, y only.

Kernel: hipo_residual_layernorm_bf16 with h, mean and rstd not written --
the row in registers, exact per-wave two-pass statistics of the
bf16-rounded h merged with Chan's formula.  Algorithmic bytes: 4 R C (x,
residual) + 4 C + 2 R C (y).
Replaces the Triton body of the reference's
repros/canonical/var_mean_80e7ff4dee7f/oracle.py:122
(_residual_layernorm_kernel, :51), without its anchor-clamp of the output.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-05


@oracle_impl(hardware="MI355X", point="1cea4d76", description="residual LN, y only")
@oracle_impl(hardware="MI355X", description="residual LN y only, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, beta, shape = inputs
    cols = x.shape[-1]
    y = hip_oracles.residual_layernorm(x.reshape(-1, cols), residual.reshape(-1, cols),
                                       gamma, beta, EPS, outputs="y")
    return y.view(shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
