"""
MI355X oracle for mean_4462ce967d63: residual add + T5 RMSNorm (HF op
order, eps 1e-6) + output scale.

Kernel: hipo_rmsnorm_ex_bf16 (mode 1, residual) -- the row in registers,
h = bf16(x + residual), fp32 sum of squares, then bf16(h * rstd),
bf16(gamma * .), bf16(. * scale) exactly in the eager op order.
Algorithmic bytes: 4 R C (x, residual) + 2 C + 2 R C (y).
Replaces the Triton body of the reference's
repros/canonical/mean_4462ce967d63/oracle.py:65.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-06
SCALE = 0.04419417382415922


@oracle_impl(hardware="MI355X", point="40057a60", description="T5 RMSNorm, rows in registers")
@oracle_impl(hardware="MI355X", description="T5 RMSNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, _shape, out_shape = inputs
    cols = x.shape[-1]
    y = hip_oracles.rmsnorm_ex(x.reshape(-1, cols), gamma, EPS,
                               residual=residual.reshape(-1, cols), scale=SCALE, mode=1)
    return y.view(out_shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
