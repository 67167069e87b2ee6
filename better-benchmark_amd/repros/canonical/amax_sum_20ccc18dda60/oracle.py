"""
MI355X oracle for amax_sum_20ccc18dda60: softmax(scores + bias) with the
bias [G, 1, Q, K] shared by the heads of each group (TrOCR attention).

Kernel: hipo_scaled_bias_softmax_bf16 (scale 1, heads = scores' head count)
-- the row in registers, the bias row of (b / heads, q) re-read from cache,
fp32 max and sum by DPP.  Algorithmic bytes: 2 B Q K (read) + 2 G Q K (bias)
+ 2 B Q K (write).
Replaces the Triton body of the reference's
repros/canonical/amax_sum_20ccc18dda60/oracle.py:63
(_broadcast_add_softmax_kernel, :12).
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", point="38831ee4", description="bias softmax, rows in registers")
@oracle_impl(hardware="MI355X", description="bias softmax, shape-general")
def oracle_forward(inputs):
    scores, bias, grouped_shape, flat_shape = inputs
    groups, heads, q, k = grouped_shape
    x = scores.reshape(flat_shape)
    return hip_oracles.scaled_bias_softmax(x, bias.reshape(bias.shape[0], q, k), 1.0, heads)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
