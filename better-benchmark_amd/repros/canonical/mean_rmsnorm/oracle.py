"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle reads x once: four waves hold each 4096-element row in registers through the fp32 sum of squares and the scaling, with non-temporal loads and stores, whereas Inductor emits triton_red_fused_add_convert_element_type_mean_mul_pow_rsqrt_0, a looped reduction whose first loop accumulates x^2 with evict_last loads and whose second loop reloads x (evict_first) and gamma to write y; Inductor cannot do this today because for rows this wide it picks a looped (non-persistent) reduction, which must walk the row twice -- the second time from cache -- instead of keeping it in registers across the statistics and the epilogue (the re-read hits in cache, so one cached launch sees the two kernels at about the same time, and a sustained stream separates them); the fix is BANDWIDTH_BOUND: a multi-wave persistent row reduction for rows of a few thousand elements that keeps the row in registers from the statistics to the epilogue, with non-temporal streams.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
0390a437, oracle 53.35 us, Inductor 51.31 us (ratio 0.962, AT_FLOOR); over the dir's 3
registered points: 3 AT_FLOOR.

MI355X oracle for mean_rmsnorm: y = x * rsqrt(mean(x^2) + eps) * gamma, rstd.

Kernel: hipo_rmsnorm_bf16 -- the row in registers (4 waves per row at
C = 4096), fp32 sum of squares reduced with DPP and a fixed-order LDS
combine, one rounding to bf16.  Algorithmic
bytes: 4 R C + 2 C + 4 R.
Replaces the Triton body of the reference's
repros/canonical/mean_4462ce967d63/oracle.py:65.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-05  # the graph constant of repro.py


@oracle_impl(hardware="MI355X", point="0390a437", description="RMSNorm, rows in registers")
@oracle_impl(hardware="MI355X", description="RMSNorm, shape-general")
def oracle_forward(inputs):
    x, gamma = inputs
    return hip_oracles.rmsnorm(x, gamma, EPS)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
