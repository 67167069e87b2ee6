"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the exact fp32 statistics of h and the LayerNorm of each row (4096 wide at the dir's largest point) with the row held in registers, reading every input once and writing y and a view of it with non-temporal 16-byte stores, whereas Inductor emits triton_red_fused_add_convert_element_type_mul_rsqrt_sub_var_mean_view_0, a looped Welford reduction that walks each row twice -- statistics, then the normalisation that reloads x and residual; Inductor cannot do this today because for rows this wide it picks a looped (non-persistent) reduction, which must walk the row twice -- the second time from cache -- instead of keeping it in registers across the statistics and the epilogue; the fix is BANDWIDTH_BOUND: a multi-wave persistent row reduction for rows of a few thousand elements that keeps the row in registers from the statistics to the epilogue, with non-temporal streams.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
d4701d13, oracle 28.0 us, Inductor 32.96 us (ratio 1.177, GOOD); over the dir's 2
registered points: 1 GOOD, 1 AT_FLOOR; 3 points withdrawn (WITHDRAWN_POINTS).

MI355X oracle for var_mean_45f7dfd4a983: residual add + LayerNorm over the
last dim (eps 1e-12), returning y and an [R, C] view of it.

Kernel: hipo_residual_layernorm_bf16 -- h = bf16(x + residual), exact fp32
statistics of the bf16 h held in registers, y = bf16((h - mean) rstd gamma +
beta); rows of 4096 take the row-length kernel (2 waves per row, gamma and
beta staged in LDS), others the row-plan kernel (W waves per row, about
2 KiB of each stream per wave).  Algorithmic bytes per row of C: 2C (x) +
2C (residual) + 2C (y).
Replaces the Triton body of the reference's
repros/canonical/var_mean_45f7dfd4a983/oracle.py:109.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-12

# Points of shapes.json with no MI355X registration.  The status sweeps
# measured Inductor more than 5 % faster at each of them (BAD_ORACLE) in the
# reference's single-launch protocol: rows of 768 or 1024 values, 16384 rows
# or more, where the two kernels are within 3 % of each other in a
# back-to-back loop but Inductor is 5-8 % faster in a single launch after a
# cache flush (layouts with 32-lane row segments, cached loads or an
# occupancy cap measured no better).  There is no shape-general
# registration, so these points find no MI355X oracle (NO_ORACLE_FOR_SHAPE,
# the reference's state of a point without one); the kernel still computes
# them and the parity tests call it directly.  Values: the measured ratios
# compile_us / oracle_us.
WITHDRAWN_POINTS = {
    "63bebcf6": (0.963, 0.949),
    "d1f40ce2": (0.945, 0.945),
    "d4cc3e3e": (0.965, 0.949),
}


@oracle_impl(hardware="MI355X", point="d4701d13",
             description="residual LayerNorm, 4096 x 4096")
@oracle_impl(hardware="MI355X", point="0b3dc49f",
             description="residual LayerNorm, 8192 x 1024")
def oracle_forward(inputs):
    x, residual, gamma, beta = inputs[:4]
    shapes = inputs[4:]
    cols = x.shape[-1]
    out = hip_oracles.residual_layernorm(x.reshape(-1, cols), residual.reshape(-1, cols),
                                         gamma, beta, EPS, outputs="y")
    y = out
    return (y.view(tuple(int(d) for d in shapes[0])),
            y.view(tuple(int(d) for d in shapes[1])))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
