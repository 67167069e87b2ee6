"""Gap diagnosis (classification: ALGEBRAIC_ELIMINATION): this oracle computes the plain attention softmax with each row held in registers (one wave per 1024-wide row, 16 lanes per 128-wide row) and the exponential evaluated once per element, whereas Inductor emits triton_per_fused_convert_element_type_div_exp_prepare_softmax_online_sub_view_0, a persistent online-softmax reduction that evaluates libdevice.exp twice per element; Inductor cannot do this today because its online-softmax lowering recomputes the exponentials rather than keeping the persistent row's exp values live; the fix is ALGEBRAIC_ELIMINATION: one exp per element for persistent rows.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
5b248c57, oracle 53.11 us, Inductor 63.99 us (ratio 1.205, GOOD); over the dir's 2
registered points: 1 AT_FLOOR, 1 GOOD.

MI355X oracle for amax_sum_fa4cc85fe5ad: the plain attention softmax of T5 /
MT5 (no bias, no scale), bf16 in and out, fp32 statistics.

Kernel: hipo_scaled_masked_softmax_bf16 with scale 1 and one zero mask row
for every row (hip_oracles.softmax_lastdim) -- K = 1024 rows go to the
shared-row kernel (the row's mask staged once per workgroup in LDS, four
rows' loads in flight per wave), K = 128 rows to the short-row kernel (16
lanes per row).  Algorithmic bytes: 2 B Q K (read) + 2 B Q K (write).
Replaces the Triton body of the reference's
repros/canonical/amax_sum_fa4cc85fe5ad/oracle.py:68 (_bf16_softmax_kernel, :12).
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main


@oracle_impl(hardware="MI355X", point="215d1cc0", description="softmax, 16 lanes per row")
@oracle_impl(hardware="MI355X", point="5b248c57", description="softmax, shared-row kernel")
@oracle_impl(hardware="MI355X", description="softmax, shape-general")
def oracle_forward(inputs):
    scores, _grouped, _expanded, flat_shape = inputs
    return hip_oracles.softmax_lastdim(scores).view(tuple(int(d) for d in flat_shape))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
