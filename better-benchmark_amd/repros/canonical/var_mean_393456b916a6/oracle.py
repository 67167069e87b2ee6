"""
MI355X oracle for var_mean_393456b916a6: residual add + LayerNorm over the
last dim (eps 1e-12), returning y and three [R, C] views of it.

Kernel: hipo_residual_layernorm_bf16 -- h = bf16(x + residual), exact fp32
statistics of the bf16 h held in registers, y = bf16((h - mean) rstd gamma +
beta); rows of 4096 take the row-length kernel (2 waves per row, gamma and
beta staged in LDS), others the row-plan kernel (W waves per row, about
2 KiB of each stream per wave).  Algorithmic bytes per row of C: 2C (x) +
2C (residual) + 2C (y).
Replaces the Triton body of the reference's
repros/canonical/var_mean_393456b916a6/oracle.py:49.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-12


@oracle_impl(hardware="MI355X", point="d4701d13",
             description="residual LayerNorm, 4096 x 4096")
@oracle_impl(hardware="MI355X", point="63bebcf6",
             description="residual LayerNorm, 16384 x 768")
@oracle_impl(hardware="MI355X", point="107053b2",
             description="residual LayerNorm, 4096 x 1536")
@oracle_impl(hardware="MI355X", point="82b81ff3",
             description="residual LayerNorm, 32768 x 768")
@oracle_impl(hardware="MI355X", point="94a8a62c",
             description="residual LayerNorm, 32768 x 256")
@oracle_impl(hardware="MI355X", description="residual LayerNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, beta = inputs[:4]
    shapes = inputs[4:]
    cols = x.shape[-1]
    out = hip_oracles.residual_layernorm(x.reshape(-1, cols), residual.reshape(-1, cols),
                                         gamma, beta, EPS, outputs="y")
    y = out
    return (y.view(tuple(int(d) for d in shapes[0])),) + tuple(
        y.view(tuple(int(d) for d in s)) for s in shapes[1:4])


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
