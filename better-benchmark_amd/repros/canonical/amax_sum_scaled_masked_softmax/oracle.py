"""Gap diagnosis (classification: ALGEBRAIC_ELIMINATION): this oracle computes the scaled, additively masked softmax with one wave per 1024-wide row held in registers, the mask row staged once in LDS for the four same-query rows of a workgroup, the exponential evaluated once per element (and not at all in 512-column groups whose scores are -inf in every lane) and the quotient taken as the IEEE division, whereas Inductor emits triton_per_fused__softmax_add_exp_mul_prepare_softmax_online_sub_0, a persistent online-softmax reduction that evaluates libdevice.exp twice per element (inside the running max / sum and again for the output) and reloads the mask row for every row; Inductor cannot do this today because its online-softmax lowering recomputes the exponentials instead of keeping a persistent row's exp values live, and it has no rule for skipping fully masked column blocks; the fix is ALGEBRAIC_ELIMINATION: keep the persistent row's exp values in registers between the sum and the normalisation (one exp per element) and skip blocks whose scores are all -inf.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
134a1d74, oracle 262.53 us, Inductor 296.85 us (ratio 1.131, GOOD); over the dir's 3
registered points: 2 AT_FLOOR, 1 GOOD.

MI355X oracle for amax_sum_scaled_masked_softmax:
softmax(scores * 0.125 + mask, -1), bf16 in/out, fp32 max and sum.

Kernel: hipo_scaled_masked_softmax_bf16 -- the row in registers (one wave
per row at K = 1024, two non-temporal 16-byte loads per lane, 8 rows per
workgroup), DPP max and sum, the [Q, K] mask row re-read from cache for
every batch entry.  Algorithmic
bytes: 2 B Q K (read) + 2 Q K (mask) + 2 B Q K (write).
Replaces the Triton body of the reference's
repros/canonical/amax_sum_20ccc18dda60/oracle.py:63.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

SCALE = 0.125  # the graph constant of repro.py


@oracle_impl(hardware="MI355X", point="134a1d74", description="masked softmax, rows in registers")
@oracle_impl(hardware="MI355X", description="masked softmax, shape-general")
def oracle_forward(inputs):
    x, mask = inputs
    return hip_oracles.scaled_masked_softmax(x, mask, SCALE)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
