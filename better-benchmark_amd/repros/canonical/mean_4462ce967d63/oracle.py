"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the fp32 sum of squares and the RMSNorm of each row (512 wide at the dir's largest point; rounding h * rstd and gamma * (.) to bf16 as the graph does) with the row held in registers, reading every input once and writing y with non-temporal 16-byte stores, whereas Inductor emits triton_per_fused_add_convert_element_type_mean_mul_pow_rsqrt_view_0, a persistent reduction that reads x, residual and gamma once with cached (evict_last) loads and writes y with cached stores; Inductor cannot do this today because its persistent reduction already reads each row once, so the gap is the access style -- one program per row block with cached evict_last loads and cached stores, against several rows per wave and non-temporal streams -- and at these sizes both sit near the memory floor; the fix is BANDWIDTH_BOUND: emit non-temporal loads and stores for single-use row tensors in the ROCm persistent-reduction template and map several short rows to one wave.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
40057a60, oracle 15.28 us, Inductor 14.6 us (ratio 0.955, NUMERICS_OPTOUT_ACCEPTED);
over the dir's 1 registered points: 1 NUMERICS_OPTOUT_ACCEPTED.

MI355X oracle for mean_4462ce967d63: residual add + T5 RMSNorm (HF op
order, eps 1e-6) + output scale.

Kernel: hipo_rmsnorm_ex_bf16 (mode 1, residual) -- the row in registers,
h = bf16(x + residual), fp32 sum of squares, then bf16(h * rstd),
bf16(gamma * .), bf16(. * scale) exactly in the eager op order.
Algorithmic bytes: 4 R C (x, residual) + 2 C + 2 R C (y).
Replaces the Triton body of the reference's
repros/canonical/mean_4462ce967d63/oracle.py:65.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-06
SCALE = 0.04419417382415922


@oracle_impl(hardware="MI355X", point="40057a60", description="T5 RMSNorm, rows in registers")
@oracle_impl(hardware="MI355X", description="T5 RMSNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma, _shape, out_shape = inputs
    cols = x.shape[-1]
    y = hip_oracles.rmsnorm_ex(x.reshape(-1, cols), gamma, EPS,
                               residual=residual.reshape(-1, cols), scale=SCALE, mode=1)
    return y.view(out_shape)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
