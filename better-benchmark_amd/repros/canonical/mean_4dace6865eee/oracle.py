"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the fp32 sum of squares and the RMSNorm of each row (512 wide at the dir's largest point; rounding h * rstd and gamma * (.) to bf16 as the graph does) with the row held in registers, reading every input once and writing y with non-temporal 16-byte stores, whereas Inductor emits triton_per_fused_add_convert_element_type_mean_mul_pow_rsqrt_view_0, a persistent reduction that reads x, residual and gamma once with cached (evict_last) loads and writes y with cached stores; Inductor cannot do this today because its persistent reduction already reads each row once, so the gap is the access style -- one program per row block with cached evict_last loads and cached stores, against several rows per wave and non-temporal streams -- and at these sizes both sit near the memory floor; the fix is BANDWIDTH_BOUND: emit non-temporal loads and stores for single-use row tensors in the ROCm persistent-reduction template and map several short rows to one wave.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
40057a60, oracle 15.12 us, Inductor 14.64 us (ratio 0.968, AT_FLOOR); over the dir's 1
registered points: 1 AT_FLOOR.

MI355X oracle for mean_4dace6865eee: residual add + RMSNorm over the last
dim (eps 1e-06), returning y and 12 views of y.

Kernel: hipo_rmsnorm_ex_bf16, mode 1 (bf16(h * rstd), then bf16(gamma * t), as the graph rounds) -- h = bf16(x +
residual) held in registers between its sum of squares and its output, W
waves per row.  Algorithmic bytes per row of C: 2C (x) + 2C (residual) +
2C (y).
Replaces the Triton body of the reference's
repros/canonical/mean_4dace6865eee/oracle.py:61.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-06


@oracle_impl(hardware="MI355X", point="40057a60",
             description="residual RMSNorm, 8192 x 512")
@oracle_impl(hardware="MI355X", description="residual RMSNorm, shape-general")
def oracle_forward(inputs):
    x, residual, gamma = inputs[:3]
    shapes = inputs[3:]
    cols = x.shape[-1]
    out = hip_oracles.rmsnorm_ex(x.reshape(-1, cols), gamma, EPS,
                                 residual=residual.reshape(-1, cols), mode=1,
                                 want_h=False)
    y = out
    return (y.view(residual.shape),
            y.view(tuple(int(d) for d in shapes[1])),
            y.view(tuple(int(d) for d in shapes[2])),
            y.view(tuple(int(d) for d in shapes[3])),
            y.view(tuple(int(d) for d in shapes[4])),
            y.view(tuple(int(d) for d in shapes[5])),
            y.view(tuple(int(d) for d in shapes[6])),
            y.view(tuple(int(d) for d in shapes[7])),
            y.view(tuple(int(d) for d in shapes[8])),
            y.view(tuple(int(d) for d in shapes[9])),
            y.view(tuple(int(d) for d in shapes[10])),
            y.view(tuple(int(d) for d in shapes[11])),
            y.view(tuple(int(d) for d in shapes[12])))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
