"""
MI355X oracle for mean_4dace6865eee: residual add + RMSNorm over the last
dim (eps 1e-06), returning y and 12 views of y.

Kernel: hipo_rmsnorm_ex_bf16, mode 1 (bf16(h * rstd), then bf16(gamma * t), as the graph rounds) -- h = bf16(x +
residual) held in registers between its sum of squares and its output, W
waves per row.  Algorithmic bytes per row of C: 2C (x) + 2C (residual) +
2C (y).
Replaces the Triton body of the reference's
repros/canonical/mean_4dace6865eee/oracle.py:61.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

EPS = 1e-06


@oracle_impl(hardware="MI355X", point="40057a60",
             description="residual RMSNorm, 8192 x 512")
@oracle_impl(hardware="MI355X", description="residual RMSNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma = inputs[:3]
    shapes = inputs[3:]
    cols = x.shape[-1]
    out = hip_oracles.rmsnorm_ex(x.reshape(-1, cols), gamma, EPS,
                                 residual=residual.reshape(-1, cols), mode=1,
                                 want_h=False)
    y = out
    return (y.view(residual.shape),
            y.view(tuple(int(d) for d in shapes[1])),
            y.view(tuple(int(d) for d in shapes[2])),
            y.view(tuple(int(d) for d in shapes[3])),
            y.view(tuple(int(d) for d in shapes[4])),
            y.view(tuple(int(d) for d in shapes[5])),
            y.view(tuple(int(d) for d in shapes[6])),
            y.view(tuple(int(d) for d in shapes[7])),
            y.view(tuple(int(d) for d in shapes[8])),
            y.view(tuple(int(d) for d in shapes[9])),
            y.view(tuple(int(d) for d in shapes[10])),
            y.view(tuple(int(d) for d in shapes[11])),
            y.view(tuple(int(d) for d in shapes[12])))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
