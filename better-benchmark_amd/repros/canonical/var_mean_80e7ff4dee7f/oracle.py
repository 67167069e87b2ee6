"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the exact fp32 statistics of h and the LayerNorm of each row (768 wide at the dir's largest point) with the row held in registers, reading every input once and writing y only with non-temporal 16-byte stores, whereas Inductor emits triton_per_fused_add_convert_element_type_mul_rsqrt_sub_var_mean_view_0, a persistent reduction with one row per program row that reads x, residual, gamma and beta once with cached (evict_last) loads and writes y only with cached stores; Inductor cannot do this today because its persistent reduction already reads each row once, so the gap is the access style -- one program per row block with cached evict_last loads and cached stores, against several rows per wave and non-temporal streams -- and at these sizes both sit near the memory floor; the fix is BANDWIDTH_BOUND: emit non-temporal loads and stores for single-use row tensors in the ROCm persistent-reduction template and map several short rows to one wave.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
1cea4d76, oracle 18.24 us, Inductor 17.0 us (ratio 0.932, BAD_ORACLE); over the dir's 1
registered points: 1 BAD_ORACLE.  The ten sweeps before measured 0.949-0.982; the
fastest oracle run against the fastest Inductor run over all eleven gives 0.959, above
the 0.95 below which a point is withdrawn, so it stays registered.  Back to back (inputs
rotating through 1.2 GB) Inductor's tuned kernel is faster at this shape, 7.65 against
8.42 us; one- or two-row workgroups and two rows per wave took 8.6-8.9 us.

MI355X oracle for var_mean_80e7ff4dee7f: residual add + LayerNorm, y only.

Kernel: hipo_residual_layernorm_bf16 with h, mean and rstd not written --
the row in registers, exact per-wave two-pass statistics of the
bf16-rounded h merged with Chan's formula.  Algorithmic bytes: 4 R C (x,
residual) + 4 C + 2 R C (y).
Replaces the Triton body of the reference's
repros/canonical/var_mean_80e7ff4dee7f/oracle.py:122
(_residual_layernorm_kernel, :51), without its anchor-clamp of the output.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-05


@oracle_impl(hardware="MI355X", point="1cea4d76", description="residual LN, y only")
@oracle_impl(hardware="MI355X", description="residual LN y only, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, beta, shape = inputs
    cols = x.shape[-1]
    y = hip_oracles.residual_layernorm(x.reshape(-1, cols), residual.reshape(-1, cols),
                                       gamma, beta, EPS, outputs="y")
    return y.view(shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
