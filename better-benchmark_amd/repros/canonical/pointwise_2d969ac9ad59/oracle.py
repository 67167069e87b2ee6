"""Gap diagnosis (classification: ALGEBRAIC_ELIMINATION): this oracle evaluates the decomposed tanh GELU as x * sigmoid(2u) -- for bf16, the correctly rounded result of every input (an fp32 exp2 / rcp form shown exact over the whole domain, an exact table below x = -4); for fp32, x / (1 + e^-2u) with an extended-precision exp and an IEEE division -- streamed as 8 KiB per wave with non-temporal accesses, whereas Inductor emits triton_poi_fused_add_mul_pow_tanh_view_0, a flat pointwise kernel that evaluates 0.5 x (1 + libdevice.tanh(u)) per element, whose 1 + tanh cancels in the negative tail; Inductor cannot do this today because it lowers aten.tanh literally and does not rewrite 0.5 x (1 + tanh(u)) into the algebraically equal, cheaper and cancellation-free x * sigmoid(2u); the fix is ALGEBRAIC_ELIMINATION: that rewrite in the pointwise lowering.

Measured on one MI355X (oracle_harness.bench_oracle: graph replay after a 1 GiB read
flush, min over rounds; Inductor with coordinate-descent tuning): at the largest point
8f687505, oracle 68.43 us, Inductor 67.27 us (ratio 0.983, AT_FLOOR); over the dir's 6
registered points: 5 GOOD, 1 AT_FLOOR.

MI355X oracle for pointwise_2d969ac9ad59: tanh GELU of a contiguous bf16 or
fp32 activation, returned in the second view's shape.

Kernels: hipo_gelu_tanh_bf16 -- the correctly rounded bf16 GELU of every
bf16 input by bit pattern (a 7 KiB table of exactly rounded results staged
in LDS, bit arithmetic outside its range; the eager graph's per-op bf16
roundings and Inductor's fp32 chain both approximate this value);
hipo_gelu_tanh_f32 -- x / (1 + e^(-2u)) with an extended-precision exp and
an IEEE division (the same function, without 1 + tanh(u)'s cancellation).  Flat streams of 16-byte non-temporal accesses,
8 KiB per wave.  Algorithmic bytes: 2 x numel x element size.
Replaces the Triton body of the reference's
repros/canonical/pointwise_2d969ac9ad59/oracle.py:44-62 (_tanh_gelu_kernel, :12).
"""
import hip_oracles
from oracle_harness import oracle_impl, oracle_main

_POINTS = ("cd47785e", "92efc45e", "d05618d1", "7b14189f", "5cd82a46", "8f687505")


def oracle_forward(inputs):
    x, _shape, out_shape = inputs
    return hip_oracles.gelu_tanh(x).view(out_shape)


for _point in _POINTS:
    oracle_forward = oracle_impl(hardware="MI355X", point=_point,
                                 description="flat tanh GELU")(oracle_forward)
oracle_forward = oracle_impl(hardware="MI355X",
                             description="flat tanh GELU, shape-general")(oracle_forward)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
