// Channel bias + GELU(tanh) fused with NCHW -> NHWC (channels-last), bf16.
//
// Tile = one wave64: 64 channels x 64 spatial positions of one image; a
// 256-thread workgroup stacks four waves over 256 channels of the same 64
// positions, so its output is one contiguous run of 64 NHWC rows.
//
// Lane l owns an 8x8 (channel x position) block: cb = l / 8 picks 8
// channels, hb = l % 8 picks 8 positions.  It issues 8 16-byte loads, one per
// channel row (the 8 lanes of equal cb read one contiguous 128-byte segment
// of that channel's row), and 8 16-byte stores, one per position (the 8 lanes
// of equal hb write one contiguous 128-byte segment of that NHWC row).  The
// 8x8 transpose happens in registers: the packed bf16 conversion
// (v_cvt_pk_bf16_f32) pairs values of adjacent channels, so no LDS staging,
// no bank conflicts and no barrier are needed for the transpose.
//
// Arithmetic is fp32 with one rounding to bf16:
//   t = x + b;  y = 0.5 t (1 + tanh(u)),  u = sqrt(2/pi) (t + 0.044715 t^3)
// evaluated as y = t / (1 + 2^(t (A + B t^2))) with A = -2 sqrt(2/pi) log2(e),
// B = 0.044715 A (the identity 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u))).
// HBM-bound: algorithmic bytes per element = 2 (read) + 2 (write).
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr float kGeluA = -2.302208198144325f;    // -2 sqrt(2/pi) log2(e)
constexpr float kGeluB = -0.1029432395800235f;   // 0.044715 * kGeluA

__device__ __forceinline__ float gelu_tanh(float t) {
  const float z = t * __builtin_fmaf(kGeluB, t * t, kGeluA);
  return t * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

constexpr int kTileHw = 64;        // positions per wave / workgroup
constexpr int kWaveC = 64;         // channels per wave
constexpr int kBlockC = 256;       // channels per workgroup (4 waves)

__global__ __launch_bounds__(256) void bias_gelu_nchw_to_nhwc_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t C, int64_t HW, int64_t hw_tiles,
    int64_t c_groups) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int64_t blk = blockIdx.x;
  const int64_t hw_tile = blk % hw_tiles;
  const int64_t rest = blk / hw_tiles;
  const int64_t cgrp = rest % c_groups;
  const int64_t img = rest / c_groups;

  const int hb = lane & 7;
  const int cb = lane >> 3;
  const int64_t c0 = cgrp * kBlockC + wave * kWaveC + cb * 8;
  const int64_t p0 = hw_tile * kTileHw + hb * 8;
  if (c0 >= C || p0 >= HW) return;  // C % 8 == 0 and HW % 8 == 0 here

  uint4 xin[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    xin[j] = *reinterpret_cast<const uint4*>(x + ((img * C + c0 + j) * HW + p0));
  }
  const uint4 bw = *reinterpret_cast<const uint4*>(bias + c0);
  const uint32_t bwords[4] = {bw.x, bw.y, bw.z, bw.w};

  // y[j][i]: channel c0 + j, position p0 + i.
  float y[8][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float b = (j & 1) ? bf16hi(bwords[j >> 1]) : bf16lo(bwords[j >> 1]);
    const uint32_t w[4] = {xin[j].x, xin[j].y, xin[j].z, xin[j].w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      y[j][2 * d] = gelu_tanh(bf16lo(w[d]) + b);
      y[j][2 * d + 1] = gelu_tanh(bf16hi(w[d]) + b);
    }
  }

#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint4 o;
    o.x = pack_bf16x2(y[0][i], y[1][i]);
    o.y = pack_bf16x2(y[2][i], y[3][i]);
    o.z = pack_bf16x2(y[4][i], y[5][i]);
    o.w = pack_bf16x2(y[6][i], y[7][i]);
    *reinterpret_cast<uint4*>(out + ((img * HW + p0 + i) * C + c0)) = o;
  }
}

// Any shape: one thread per output element, NHWC order (coalesced stores,
// strided loads).
__global__ __launch_bounds__(256) void bias_gelu_nchw_to_nhwc_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t N, int64_t C, int64_t HW) {
  const int64_t total = N * C * HW;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       o < total; o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = o % C;
    const int64_t p = (o / C) % HW;
    const int64_t img = o / (C * HW);
    const float t = bf16_to_f32(x[(img * C + c) * HW + p]) + bf16_to_f32(bias[c]);
    out[o] = static_cast<uint16_t>(pack_bf16x2(gelu_tanh(t), 0.0f) & 0xffffu);
  }
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_bias_gelu_nchw_to_nhwc_bf16(const uint16_t* x,
                                                const uint16_t* bias,
                                                uint16_t* out, int64_t n,
                                                int64_t c, int64_t hw,
                                                hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n >= 0 && c >= 0 && hw >= 0, "bias_gelu: negative size");
  if (n == 0 || c == 0 || hw == 0) return 0;
  HIPO_REQUIRE(x && bias && out, "bias_gelu: null pointer");
  const bool vec = (c % 8 == 0) && (hw % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(bias) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  if (vec) {
    const int64_t hw_tiles = (hw + kTileHw - 1) / kTileHw;
    const int64_t c_groups = (c + kBlockC - 1) / kBlockC;
    const int64_t blocks = n * c_groups * hw_tiles;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "bias_gelu: grid too large");
    bias_gelu_nchw_to_nhwc_vec<<<dim3(static_cast<unsigned>(blocks)), dim3(256),
                                 0, stream>>>(x, bias, out, c, hw, hw_tiles,
                                              c_groups);
  } else {
    const int64_t total = n * c * hw;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    bias_gelu_nchw_to_nhwc_scalar<<<dim3(static_cast<unsigned>(blocks)),
                                    dim3(256), 0, stream>>>(x, bias, out, n, c,
                                                            hw);
  }
  return check_launch("bias_gelu_nchw_to_nhwc_bf16");
}
