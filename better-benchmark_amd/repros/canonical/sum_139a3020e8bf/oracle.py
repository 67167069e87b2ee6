"""Gap diagnosis (classification: SCHEDULER_FUSION): this oracle writes the erf-GELU gradient y = bf16(grad * GELU'(x)) and accumulates its column sums from the bf16 y in the same pass (GELU'(x) from an LDS table of its correctly rounded fp32 value at every bf16 x; fp32 partials per row block, then a second launch adds them in a fixed order), whereas Inductor emits three kernels -- triton_poi_fused_add_convert_element_type_erf_exp_mul_view_0 writing y (libdevice.erf and exp per element), then two reduction kernels that read y back to form the column sums; Inductor cannot do this today because the scheduler does not fuse a column (dim-0) reduction into the pointwise kernel that produces its input when the pointwise output is also returned; the fix is SCHEDULER_FUSION: fuse the producer with a split column reduction that accumulates from registers.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
3f451298, oracle 552.38 us, Inductor 759.91 us (ratio 1.376, GOOD); over the dir's 14
registered points: 14 GOOD; 1 points withdrawn (WITHDRAWN_POINTS).

MI355X oracle for sum_139a3020e8bf: the gradient through an erf GELU, y = bf16(grad *
GELU'(x)), returned with its transpose view, and its column sum (the bias
gradient) rounded to bf16 and stored as fp32.

Kernel: hipo_gelu_erf_bwd_colsum_bf16 -- GELU'(x) read from an LDS table of
its correctly rounded fp32 value at every bf16 x, one fp32 product per
element, y written once and its column partials accumulated from the bf16 y
in the same pass (fp32, one row per row block), then a second launch adds
the partials in a fixed order.  Algorithmic bytes: 2 R C (grad) + 2 R C (x)
+ 2 R C (y) + 4 C (colsum).
Replaces the Triton body of the reference's
repros/canonical/sum_139a3020e8bf/oracle.py:101.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

# Points of shapes.json with no MI355X registration: [128, 3072] (0.8 MB),
# one launch of 48 workgroups at the graph-replay floor, where the oracle
# holds 15.0-15.1 us and Inductor's re-tuned kernels took 14.3-16.7 us
# across the status sweeps (BAD_ORACLE in two of three).  There is no
# shape-general registration, so the point finds no MI355X oracle
# (NO_ORACLE_FOR_SHAPE); the kernel still computes it and the parity tests
# call it directly.  Values: the measured ratios compile_us / oracle_us.
WITHDRAWN_POINTS = {
    "67c7a377": (1.115, 0.952, 0.944),
}


@oracle_impl(hardware="MI355X", point="8572c66c",
             description="GELU(erf) bwd + column sum, 25216 x 3072")
@oracle_impl(hardware="MI355X", point="9448cee8",
             description="GELU(erf) bwd + column sum, 25216 x 768")
@oracle_impl(hardware="MI355X", point="5c6c31bb",
             description="GELU(erf) bwd + column sum, 25344 x 3072")
@oracle_impl(hardware="MI355X", point="3f451298",
             description="GELU(erf) bwd + column sum, 175360 x 3072")
@oracle_impl(hardware="MI355X", point="c064ba70",
             description="GELU(erf) bwd + column sum, 32768 x 3072")
@oracle_impl(hardware="MI355X", point="8951d544",
             description="GELU(erf) bwd + column sum, 8192 x 4096")
@oracle_impl(hardware="MI355X", point="a448a1c6",
             description="GELU(erf) bwd + column sum, 4096 x 10240")
@oracle_impl(hardware="MI355X", point="5d96adde",
             description="GELU(erf) bwd + column sum, 2048 x 10240")
@oracle_impl(hardware="MI355X", point="63ec809a",
             description="GELU(erf) bwd + column sum, 4096 x 6144")
@oracle_impl(hardware="MI355X", point="05a5e903",
             description="GELU(erf) bwd + column sum, 16384 x 3072")
@oracle_impl(hardware="MI355X", point="7c6aa97f",
             description="GELU(erf) bwd + column sum, 32768 x 1024")
@oracle_impl(hardware="MI355X", point="58ff2bc5",
             description="GELU(erf) bwd + column sum, 8192 x 3072")
@oracle_impl(hardware="MI355X", point="6a0c3b2c",
             description="GELU(erf) bwd + column sum, 16384 x 4096")
@oracle_impl(hardware="MI355X", point="7c4310e0",
             description="GELU(erf) bwd + column sum, 4096 x 4096")
def oracle_forward(inputs):
    grad, x, _shape0, _shape1, shape2, shape3 = inputs
    rows, cols = int(shape2[0]), int(shape2[1])
    y, colsum = hip_oracles.gelu_erf_bwd_colsum(grad.view(rows, cols), x.view(rows, cols))
    return (y, y.permute(1, 0), colsum.view(tuple(int(d) for d in shape3)))


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
