"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the fp32 sum of squares and the RMSNorm of each row (2880 wide at the dir's largest point; rounding gamma * h * rstd to bf16 once) with the row held in registers, reading every input once and writing h and y with non-temporal 16-byte stores, whereas Inductor emits triton_red_fused_add_convert_element_type_mean_mul_pow_rsqrt_view_0, a looped reduction whose first loop forms h and its sum of squares and whose second loop reloads the inputs to write h and y; Inductor cannot do this today because for rows this wide it picks a looped (non-persistent) reduction, which must walk the row twice -- the second time from cache -- instead of keeping it in registers across the statistics and the epilogue; the fix is BANDWIDTH_BOUND: a multi-wave persistent row reduction for rows of a few thousand elements that keeps the row in registers from the statistics to the epilogue, with non-temporal streams.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
533b2091, oracle 15.8 us, Inductor 15.92 us (ratio 1.008, AT_FLOOR); over the dir's 1
registered points: 1 AT_FLOOR.

MI355X oracle for mean_f21cc667fe83: residual add + RMSNorm over the last
dim (eps 1e-05), returning the bf16 sum h and 1 view of y.

Kernel: hipo_rmsnorm_ex_bf16, mode 0 (bf16(gamma * h * rstd), one rounding) -- h = bf16(x +
residual) held in registers between its sum of squares and its output, W
waves per row.  Algorithmic bytes per row of C: 2C (x) + 2C (residual) +
2C (y) + 2C (h).
Replaces the Triton body of the reference's
repros/canonical/mean_f21cc667fe83/oracle.py:56.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-05


@oracle_impl(hardware="MI355X", point="533b2091",
             description="residual RMSNorm, 1000 x 2880")
@oracle_impl(hardware="MI355X", description="residual RMSNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma = inputs[:3]
    shapes = inputs[3:]
    cols = x.shape[-1]
    out = hip_oracles.rmsnorm_ex(x.reshape(-1, cols), gamma, EPS,
                                 residual=residual.reshape(-1, cols), mode=0,
                                 want_h=True)
    h, y = out
    return (h.view(residual.shape),
            y.view(tuple(int(d) for d in shapes[1])))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
