"""
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
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", point="8d22dcbf", description="bias+gelu NCHW->NHWC, register transpose")
@oracle_impl(hardware="MI355X", description="bias+gelu NCHW->NHWC, shape-general")
def oracle_forward(inputs):
    x, bias = inputs
    return hip_oracles.bias_gelu_nchw_to_nhwc(x, bias)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
