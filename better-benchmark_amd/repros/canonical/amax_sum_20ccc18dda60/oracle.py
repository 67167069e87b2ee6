"""Gap diagnosis (classification: NEW_PATTERN): this oracle computes softmax(scores + bias) over 256-wide rows with 16 lanes per row holding it in registers (four rows per wave instruction, segmented DPP reductions, the group's bias row read from cache) and reads the scores once, whereas Inductor emits triton_red_fused_add_convert_element_type_div_exp_prepare_softmax_online_sub_view_0, a looped reduction that walks each row twice -- an online max / sum pass and an output pass that reloads scores and bias and evaluates exp again; Inductor cannot do this today because for this shape its heuristics pick a non-persistent reduction and have no several-rows-per-wave layout for short rows; the fix is NEW_PATTERN: a short-row softmax template (several rows per wave, the row in registers, one exp per element).

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
38831ee4, oracle 56.71 us, Inductor 119.35 us (ratio 2.104, GOOD); over the dir's 1
registered points: 1 GOOD.

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
import hip_oracles
from oracle_harness import oracle_impl, oracle_main


@oracle_impl(hardware="MI355X", point="38831ee4", description="bias softmax, rows in registers")
@oracle_impl(hardware="MI355X", description="bias softmax, shape-general")
def oracle_forward(inputs):
    scores, bias, grouped_shape, flat_shape = inputs
    groups, heads, q, k = grouped_shape
    x = scores.reshape(flat_shape)
    return hip_oracles.scaled_bias_softmax(x, bias.reshape(bias.shape[0], q, k), 1.0, heads)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
