"""
MI355X oracle for mean_8818e35b12aa: residual add + RMSNorm over the last
dim (eps 1e-06), returning the bf16 sum h and 1 view of y.

Kernel: hipo_rmsnorm_ex_bf16, mode 1 (bf16(h * rstd), then bf16(gamma * t), as the graph rounds) -- h = bf16(x +
residual) held in registers between its sum of squares and its output, W
waves per row.  Algorithmic bytes per row of C: 2C (x) + 2C (residual) +
2C (y) + 2C (h).
Replaces the Triton body of the reference's
repros/canonical/mean_8818e35b12aa/oracle.py:65.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-06


@oracle_impl(hardware="MI355X", point="841ed042",
             description="residual RMSNorm, 4096 x 512")
@oracle_impl(hardware="MI355X", point="40057a60",
             description="residual RMSNorm, 8192 x 512")
@oracle_impl(hardware="MI355X", description="residual RMSNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma = inputs[:3]
    shapes = inputs[3:]
    cols = x.shape[-1]
    out = hip_oracles.rmsnorm_ex(x.reshape(-1, cols), gamma, EPS,
                                 residual=residual.reshape(-1, cols), mode=1,
                                 want_h=True)
    h, y = out
    return (h.view(residual.shape),
            y.view(tuple(int(d) for d in shapes[1])))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
