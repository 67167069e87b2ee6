// Channel bias + GELU(tanh) fused with NCHW -> NHWC (channels-last), bf16.
//
// Semantics (the eager op order of gelu(x + bias) on bf16 tensors):
//   t = bf16(x + bias[c])            (fp32 add, round to nearest even)
//   y = bf16(GELU_tanh(t))           (fp32 arithmetic, one rounding)
// GELU_tanh(t) = 0.5 t (1 + tanh(u)), u = sqrt(2/pi) (t + 0.044715 t^3), is
// evaluated as the same function in the form
//   t * sigmoid(2u) = t / (1 + 2^z),   z = t * (K0 + K1 t^2),
//   K0 = -2 sqrt(2/pi) log2(e),  K1 = 0.044715 K0,
// with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32): one FMA,
// three multiplies, one add and two transcendentals per value.  This form
// keeps the small negative tail that 1 + tanh(u) cancels to zero, gives
// +inf at +inf and NaN at -inf (as -inf * 0 in the tanh form), and rounds to
// the same bf16 as the correctly rounded function except within a few fp32
// ulps of a bf16 rounding boundary.
//
// Layout: one wave64 per tile of 64 channels x 64 spatial positions of one
// image.  Lane l owns an 8x8 (channel x position) block: cb = l / 8 picks 8
// channels, hb = l % 8 picks 8 positions.  It issues 8 16-byte loads, one
// per channel row (the 8 lanes of equal cb read one contiguous 128-byte
// segment of that row), and 8 16-byte stores, one per position (the 8 lanes
// of equal hb write one contiguous 128-byte segment of that NHWC row); the
// 8x8 transpose happens in registers, with no LDS and no barrier.  Tiles are
// numbered channel group fastest, then position tile, then image; a 256-
// thread workgroup takes four consecutive tiles (with C = 256: all channel
// groups of one position tile, i.e. 64 whole NHWC rows).  The grid is one-
// shot (no persistent loop): on MI355X many short workgroups dispatched in
// order keep the chip's in-flight address window compact, which measured
// 67.5 us for config 2 against 71 us for a persistent one-workgroup-per-CU
// version of this kernel with the GELU read from a 128 KiB LDS table.
// Loads and stores are non-temporal.
// HBM-bound: algorithmic bytes per element = 2 (read) + 2 (write).
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kTileHw = 64;  // positions per wave tile
constexpr int kTileC = 64;   // channels per wave tile
constexpr int kWavesPerBlock = 4;
constexpr int kBlockThreads = kWavesPerBlock * kWave;

constexpr float kGeluK0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
constexpr float kGeluK1 = kGeluK0 * 0.044715f;

__device__ __forceinline__ float gelu_tanh_f32(float t) {
  const float z = t * __builtin_fmaf(kGeluK1, t * t, kGeluK0);
  return t * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

struct TileGeom {
  int64_t C, HW;
  int c_tiles, hw_tiles, ntiles;  // ntiles < 2^31 (checked on the host)
};

// GRID3: the grid carries the tile coordinates (x = group of kWavesPerBlock
// channel tiles, y = position tile, z = image), so a workgroup starts its
// loads without integer divisions (66.1 against 66.6 us at config 2); the
// dispatch order is the 1-D numbering's.  Otherwise (grids past the y / z
// limits) the block index is split by division.
template <bool GRID3>
__global__ __launch_bounds__(kBlockThreads) void bias_gelu_nchw_to_nhwc_tiles(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, TileGeom g) {
  const int lane = threadIdx.x & (kWave - 1);
  int ct, ht;
  int64_t img;
  if constexpr (GRID3) {
    ct = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kWavesPerBlock +
                                        static_cast<int>(threadIdx.x >> 6));
    if (ct >= g.c_tiles) return;  // wave-uniform; the kernel has no barrier
    ht = blockIdx.y;
    img = blockIdx.z;
  } else {
    const int t = __builtin_amdgcn_readfirstlane(
        static_cast<int>(blockIdx.x) * kWavesPerBlock + static_cast<int>(threadIdx.x >> 6));
    if (t >= g.ntiles) return;  // wave-uniform
    ct = t % g.c_tiles;
    const int rest = t / g.c_tiles;
    ht = rest % g.hw_tiles;
    img = rest / g.hw_tiles;
  }
  const int64_t c0 = static_cast<int64_t>(ct) * kTileC + (lane >> 3) * 8;
  const int64_t p0 = static_cast<int64_t>(ht) * kTileHw + (lane & 7) * 8;
  // Lanes outside a partial tile load from the tile's first block (always in
  // bounds, no branch around the loads) and store nothing.
  const bool ok = c0 < g.C && p0 < g.HW;
  const int64_t cl = ok ? c0 : static_cast<int64_t>(ct) * kTileC;
  const int64_t pl = ok ? p0 : static_cast<int64_t>(ht) * kTileHw;
  const int64_t in_off = (img * g.C + cl) * g.HW + pl;

  u32x4_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    v[j] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(x + in_off + j * g.HW));
  const u32x4_t bw = *reinterpret_cast<const u32x4_t*>(bias + cl);
  float b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = (j & 1) ? bf16hi(bw[j >> 1]) : bf16lo(bw[j >> 1]);

  if (!ok) return;
  const int64_t out_off = (img * g.HW + p0) * g.C + c0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // Position p0 + i, channels c0 .. c0 + 7: round t for two channels into
    // one word (v_cvt_pk_bf16_f32), GELU both halves, pack the results.
    u32x4_t o;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t w0 = v[2 * k][i >> 1];
      const uint32_t w1 = v[2 * k + 1][i >> 1];
      const float x0 = (i & 1) ? bf16hi(w0) : bf16lo(w0);
      const float x1 = (i & 1) ? bf16hi(w1) : bf16lo(w1);
      const uint32_t tt = pack_bf16x2(x0 + b[2 * k], x1 + b[2 * k + 1]);
      o[k] = pack_bf16x2(gelu_tanh_f32(bf16lo(tt)), gelu_tanh_f32(bf16hi(tt)));
    }
    __builtin_nontemporal_store(
        o, reinterpret_cast<u32x4_t*>(out + out_off + static_cast<int64_t>(i) * g.C));
  }
}

// Any shape: one thread per output element, NHWC order (coalesced stores,
// strided loads); same arithmetic as the tile kernel.
__global__ __launch_bounds__(256) void bias_gelu_nchw_to_nhwc_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t N, int64_t C, int64_t HW) {
  const int64_t total = N * C * HW;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       o < total; o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = o % C;
    const int64_t p = (o / C) % HW;
    const int64_t img = o / (C * HW);
    const float t =
        round_bf16(bf16_to_f32(x[(img * C + c) * HW + p]) + bf16_to_f32(bias[c]));
    out[o] = static_cast<uint16_t>(pack_bf16x2(gelu_tanh_f32(t), 0.0f) & 0xffffu);
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
  const bool vec = (c % 8 == 0) && (hw % 8 == 0) && aligned16(x) &&
                   aligned16(bias) && aligned16(out);
  if (vec) {
    const int64_t c_tiles = (c + kTileC - 1) / kTileC;
    const int64_t hw_tiles = (hw + kTileHw - 1) / kTileHw;
    const int64_t ntiles = n * c_tiles * hw_tiles;
    HIPO_REQUIRE(ntiles < (int64_t{1} << 31) - kWavesPerBlock,
                 "bias_gelu: %lld tiles exceed the 32-bit tile index",
                 (long long)ntiles);
    TileGeom g;
    g.C = c;
    g.HW = hw;
    g.c_tiles = static_cast<int>(c_tiles);
    g.hw_tiles = static_cast<int>(hw_tiles);
    g.ntiles = static_cast<int>(ntiles);
    const int64_t c_groups = (c_tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (hw_tiles <= 65535 && n <= 65535) {
      const dim3 grid(static_cast<unsigned>(c_groups), static_cast<unsigned>(hw_tiles),
                      static_cast<unsigned>(n));
      bias_gelu_nchw_to_nhwc_tiles<true><<<grid, dim3(kBlockThreads), 0, stream>>>(x, bias, out,
                                                                                  g);
    } else {
      const int64_t blocks = (ntiles + kWavesPerBlock - 1) / kWavesPerBlock;
      bias_gelu_nchw_to_nhwc_tiles<false><<<dim3(static_cast<unsigned>(blocks)),
                                            dim3(kBlockThreads), 0, stream>>>(x, bias, out, g);
    }
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
