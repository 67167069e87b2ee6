"""Gap diagnosis (classification: NEW_PATTERN): this oracle fuses the channel-bias add, the tanh GELU and the NCHW -> channels-last transpose into one pass in which each lane transposes an 8 x 8 channel-by-position block in registers, so the loads and the stores are both 16-byte accesses forming 128-byte segments, and it returns the correctly rounded bf16 GELU of every bf16 input (an fp32 exp2 / rcp form shown exact over the whole domain, an exact table below t = -4) instead of evaluating tanh, whereas Inductor emits triton_poi_fused_add_clone_gelu_view_0, a Grid2D tiled pointwise kernel that loads NCHW rows with cached evict_last loads, evaluates libdevice.tanh per element and stores to the transposed index; Inductor cannot do this today because its pointwise codegen has no register-transpose tiling for a layout-changing store and lowers GELU-tanh through libdevice.tanh, whose instruction count leaves the kernel VALU-bound on gfx950 without packed fp32 math; the fix is NEW_PATTERN: a transposing pointwise template with per-lane 8 x 8 register blocks and 16-byte accesses on both sides, plus a tanh-free x * sigmoid(2u) lowering of GELU-tanh.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
8d22dcbf, oracle 76.47 us, Inductor 93.63 us (ratio 1.224, GOOD); over the dir's 3
registered points: 2 AT_FLOOR, 1 GOOD.

MI355X oracle for pointwise_bias_gelu_tanh_nhwc:
gelu_tanh(x + bias[None, :, None, None]) written channels-last (bf16).

Kernel: hipo_bias_gelu_nchw_to_nhwc_bf16 -- one pass; each lane transposes
an 8x8 (channel x position) block in registers so both the NCHW loads and
the NHWC stores are 16-byte accesses that form 128-byte contiguous
segments.  fp32 arithmetic, one rounding to bf16.  Algorithmic bytes:
2 N C H W (read) + 2 C (bias) + 2 N C H W (write).
Replaces the Triton bodies of the reference's
repros/canonical/pointwise_2d969ac9ad59/oracle.py:47 and
repros/canonical/pointwise_021e90d9c17d/oracle.py:58.
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main


@oracle_impl(hardware="MI355X", point="8d22dcbf", description="bias+gelu NCHW->NHWC, register transpose")
@oracle_impl(hardware="MI355X", description="bias+gelu NCHW->NHWC, shape-general")
def oracle_forward(inputs):
    x, bias = inputs
    return hip_oracles.bias_gelu_nchw_to_nhwc(x, bias)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
