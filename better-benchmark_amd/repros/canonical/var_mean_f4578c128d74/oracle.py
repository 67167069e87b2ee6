"""Gap diagnosis (classification: BANDWIDTH_BOUND): this oracle computes h = bf16(x + residual), the exact fp32 statistics of h and the LayerNorm of each row (768 wide at the dir's largest point) with the row held in registers, reading every input once and writing h and y with non-temporal 16-byte stores, whereas Inductor emits triton_per_fused_add_convert_element_type_mul_rsqrt_sub_var_mean_view_0, a persistent reduction with one row per program row that reads x, residual, gamma and beta once with cached (evict_last) loads and writes h and y with cached stores; Inductor cannot do this today because its persistent reduction already reads each row once, so the gap is the access style -- one program per row block with cached evict_last loads and cached stores, against several rows per wave and non-temporal streams -- and at these sizes both sit near the memory floor; the fix is BANDWIDTH_BOUND: emit non-temporal loads and stores for single-use row tensors in the ROCm persistent-reduction template and map several short rows to one wave.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
c4bf51cc, oracle 28.28 us, Inductor 29.6 us (ratio 1.047, AT_FLOOR); over the dir's 11
registered points: 9 AT_FLOOR, 2 GOOD; 5 points withdrawn (WITHDRAWN_POINTS).

MI355X oracle for var_mean_f4578c128d74: residual add + LayerNorm over the
last dim (eps 1e-06), returning the bf16 sum h and y.

Kernel: hipo_residual_layernorm_bf16 -- h = bf16(x + residual), exact fp32
statistics of the bf16 h held in registers, y = bf16((h - mean) rstd gamma +
beta); rows of 4096 take the row-length kernel (2 waves per row, gamma and
beta staged in LDS), others the row-plan kernel (W waves per row, about
2 KiB of each stream per wave).  Algorithmic bytes per row of C: 2C (x) +
2C (residual) + 2C (y) + 2C (h).
Replaces the Triton body of the reference's
repros/canonical/var_mean_f4578c128d74/oracle.py:74.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

EPS = 1e-06

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
# [131072, 144] (rows of 144 values, no row-class relation to the above):
# the oracle held 36.7-37.1 us in seven sweeps while Inductor's re-tuned
# kernel took 34.6-38.2 us; its fastest beats the oracle's fastest by 5.8 %.
WITHDRAWN_POINTS = {
    "d8c968d2": (1.017, 1.019, 1.03, 1.014, 1.013, 0.997, 0.938),
    "155170ab": (0.956, 0.989, 0.977, 0.961),
    "9801ab6a": (0.927, 0.959),
    "63bebcf6": (0.980, 0.993, 0.993, 0.981),
    "a3e95c29": (0.988, 0.951, 0.972, 0.940),
}


@oracle_impl(hardware="MI355X", point="ad6d6241",
             description="residual LayerNorm, 25216 x 192")
@oracle_impl(hardware="MI355X", point="a2357153",
             description="residual LayerNorm, 8192 x 240")
@oracle_impl(hardware="MI355X", point="f049abfe",
             description="residual LayerNorm, 32768 x 192")
@oracle_impl(hardware="MI355X", point="c4bf51cc",
             description="residual LayerNorm, 4096 x 2560")
@oracle_impl(hardware="MI355X", point="7f824027",
             description="residual LayerNorm, 2048 x 2560")
@oracle_impl(hardware="MI355X", point="1cea4d76",
             description="residual LayerNorm, 8192 x 768")
@oracle_impl(hardware="MI355X", point="17affd46",
             description="residual LayerNorm, 8192 x 1024")
@oracle_impl(hardware="MI355X", point="0b3dc49f",
             description="residual LayerNorm, 8192 x 1024")
@oracle_impl(hardware="MI355X", point="ceab07f0",
             description="residual LayerNorm, 8192 x 1024")
@oracle_impl(hardware="MI355X", point="f2e11670",
             description="residual LayerNorm, 4096 x 1024")
@oracle_impl(hardware="MI355X", point="324149d9",
             description="residual LayerNorm, 1 x 384")
def oracle_forward(inputs):
    x, residual, gamma, beta = inputs[:4]
    shapes = inputs[4:]
    cols = x.shape[-1]
    out = hip_oracles.residual_layernorm(x.reshape(-1, cols), residual.reshape(-1, cols),
                                         gamma, beta, EPS, outputs="hy")
    h, y = out
    return h.view(residual.shape), y.view(tuple(int(d) for d in shapes[1]))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
