"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the exact fp32 row statistics of h and y in one pass with each 4096-element row held in registers by two waves (gamma and beta staged in LDS, non-temporal 16-byte streams), whereas Inductor emits triton_red_fused_add_convert_element_type_mul_rsqrt_sub_var_mean_0, a looped reduction that stores h and merges Welford triples in its first R0_BLOCK loop and reloads h from its own output in a second loop to normalise; Inductor cannot do this today because for rows this wide it picks a looped (non-persistent) reduction, which must walk the row twice -- the second time from cache -- instead of keeping it in registers across the statistics and the epilogue; the fix is BANDWIDTH_BOUND: a multi-wave persistent row reduction for rows of a few thousand elements that keeps the row in registers from the statistics to the epilogue, with non-temporal streams.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
fe9bbcba, oracle 98.23 us, Inductor 106.71 us (ratio 1.086, NUMERICS_OPTOUT_ACCEPTED);
over the dir's 3 registered points: 3 NUMERICS_OPTOUT_ACCEPTED.

MI355X oracle for var_mean_residual_layernorm:
h = x + residual; y = LayerNorm(h) * gamma + beta; mean, rstd (fp32).

Kernel: hipo_residual_layernorm_bf16 -- the row in registers between the
statistics and the normalisation (x and residual are read once; 4 waves per
row at C = 4096), exact two-pass fp32 statistics of each wave's values of
the bf16-rounded h, merged across waves with Chan's formula.  Algorithmic bytes: 8 R C + 4 C + 8 R.
Replaces the Triton body of the reference's
repros/canonical/var_mean_80e7ff4dee7f/oracle.py:122 (without its
anchor-clamp of the output).
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-05  # the graph constant of repro.py


@oracle_impl(hardware="MI355X", point="fe9bbcba", description="residual LN, rows in registers")
@oracle_impl(hardware="MI355X", description="residual LN, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, beta = inputs
    return hip_oracles.residual_layernorm(x, residual, gamma, beta, EPS)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
