"""
MI355X oracle for var_mean_ee167627f636: residual add + LayerNorm over the
last dim (eps 1e-05), returning y only (viewed [R, C]).

Kernel: hipo_residual_layernorm_bf16 -- h = bf16(x + residual), exact fp32
statistics of the bf16 h held in registers, y = bf16((h - mean) rstd gamma +
beta); rows of 4096 take the row-length kernel (2 waves per row, gamma and
beta staged in LDS), others the row-plan kernel (W waves per row, about
2 KiB of each stream per wave).  Algorithmic bytes per row of C: 2C (x) +
2C (residual) + 2C (y).
Replaces the Triton body of the reference's
repros/canonical/var_mean_ee167627f636/oracle.py:114.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-05


@oracle_impl(hardware="MI355X", point="e4faf4aa",
             description="residual LayerNorm, 8192 x 768")
@oracle_impl(hardware="MI355X", description="residual LayerNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, beta = inputs[:4]
    shapes = inputs[4:]
    cols = x.shape[-1]
    out = hip_oracles.residual_layernorm(x.reshape(-1, cols), residual.reshape(-1, cols),
                                         gamma, beta, EPS, outputs="y")
    y = out
    return y.view(tuple(int(d) for d in shapes[-1]))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
