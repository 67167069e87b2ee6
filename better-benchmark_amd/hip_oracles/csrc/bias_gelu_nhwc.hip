// Channel bias + GELU(tanh) fused with NCHW -> NHWC (channels-last), bf16.
//
// Semantics (the eager op order of gelu(x + bias) on bf16 tensors):
//   t = bf16(x + bias[c])            (fp32 add, round to nearest even)
//   y = bf16(GELU_tanh(t))           (fp32 arithmetic, one rounding)
// GELU_tanh(t) = 0.5 t (1 + tanh(u)), u = sqrt(2/pi) (t + 0.044715 t^3).
// t is a bf16 value, so the output is a function of its 65536 bit patterns,
// and the kernel returns the correctly rounded bf16 of the exact function
// (gelu_bf16.h: an fp32 evaluation for t > -4 that rounds correctly for
// every such bf16 t, the exact table in global memory below that).
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
// order keep the chip's in-flight address window compact (a persistent
// one-workgroup-per-CU version of this kernel ran 71 us at config 2).  The
// kernel uses no LDS and has no barrier: a 7 KiB table staged into LDS by
// every workgroup cost 3-5 us at config 2 (25,088 waves, each waiting at the
// barrier for the table before its first lookup).
// Loads and stores are non-temporal.  Launches of at most 2^19 elements
// (and shapes off the 16-byte vector path) take a one-element-per-thread
// kernel instead.
// HBM-bound: algorithmic bytes per element = 2 (read) + 2 (write).
#include "gelu_bf16.h"
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kTileHw = 64;  // positions per wave tile
constexpr int kTileC = 64;   // channels per wave tile
constexpr int kWavesC = 4;  // waves of a workgroup along channels (consecutive channel tiles)
constexpr int kWavesP = 1;  // and along positions (consecutive position tiles)
constexpr int kWavesPerBlock = kWavesC * kWavesP;
constexpr int kBlockThreads = kWavesPerBlock * kWave;
constexpr int kTilesPerWave = 1;  // consecutive position tiles per wave (3-D grid)
constexpr int64_t kTileMinElems = int64_t{1} << 19;  // smaller launches: scalar kernel

struct TileGeom {
  int64_t C, HW;
  int c_tiles, hw_tiles, ntiles;  // ntiles < 2^31 (checked on the host)
};

// GRID3: the grid carries the tile coordinates (x = group of kWavesC channel
// tiles, y = group of kWavesP x TPW position tiles, z = image), so a workgroup starts its
// loads without integer divisions (66.1 against 66.6 us at config 2); the
// dispatch order is the 1-D numbering's.  Otherwise (grids past the y / z
// limits) the block index is split by division.
template <bool GRID3, int TPW>
__global__ __launch_bounds__(kBlockThreads) void bias_gelu_nchw_to_nhwc_tiles(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, TileGeom g) {
  const int lane = threadIdx.x & (kWave - 1);
  int ct, ht0;
  int64_t img;
  bool tile_ok;  // wave-uniform
  if constexpr (GRID3) {
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    ct = static_cast<int>(blockIdx.x) * kWavesC + wave % kWavesC;
    ht0 = (static_cast<int>(blockIdx.y) * kWavesP + wave / kWavesC) * TPW;
    tile_ok = ct < g.c_tiles && ht0 < g.hw_tiles;
    if (!tile_ok) ct = 0, ht0 = 0;
    img = blockIdx.z;
  } else {
    static_assert(GRID3 || TPW == 1, "the 1-D numbering takes one tile per wave");
    int t = __builtin_amdgcn_readfirstlane(
        static_cast<int>(blockIdx.x) * kWavesPerBlock + static_cast<int>(threadIdx.x >> 6));
    tile_ok = t < g.ntiles;
    if (!tile_ok) t = 0;
    ct = t % g.c_tiles;
    const int rest = t / g.c_tiles;
    ht0 = rest % g.hw_tiles;
    img = rest / g.hw_tiles;
  }
  const int64_t c0 = static_cast<int64_t>(ct) * kTileC + (lane >> 3) * 8;
  // Lanes outside a partial tile load from the tile's first block (always in
  // bounds, no branch around the loads) and store nothing.
  const bool c_ok = tile_ok && c0 < g.C;
  const int64_t cl = c_ok ? c0 : static_cast<int64_t>(ct) * kTileC;

  auto load_tile = [&](int ht, u32x4_t (&v)[8]) {
    const int64_t p0 = static_cast<int64_t>(ht) * kTileHw + (lane & 7) * 8;
    const int64_t pl = p0 < g.HW ? p0 : static_cast<int64_t>(ht) * kTileHw;
    const int64_t in_off = (img * g.C + cl) * g.HW + pl;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(x + in_off + j * g.HW));
  };

  u32x4_t va[8], vb[8];
  load_tile(ht0, va);
  const u32x4_t bw = *reinterpret_cast<const u32x4_t*>(bias + cl);
  float b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = (j & 1) ? bf16hi(bw[j >> 1]) : bf16lo(bw[j >> 1]);

  auto gelu_store = [&](int ht, const u32x4_t (&v)[8]) {
    const int64_t p0 = static_cast<int64_t>(ht) * kTileHw + (lane & 7) * 8;
    if (!c_ok || p0 >= g.HW) return;
    const int64_t out_off = (img * g.HW + p0) * g.C + c0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // Position p0 + i, channels c0 .. c0 + 7: round t for two channels
      // into one word (v_cvt_pk_bf16_f32), map both halves, pack them.
      u32x4_t o, tt;
      bool rare = false;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t w0 = v[2 * k][i >> 1];
        const uint32_t w1 = v[2 * k + 1][i >> 1];
        const float x0 = (i & 1) ? bf16hi(w0) : bf16lo(w0);
        const float x1 = (i & 1) ? bf16hi(w1) : bf16lo(w1);
        tt[k] = pack_bf16x2(x0 + b[2 * k], x1 + b[2 * k + 1]);
        o[k] = gelu_pair_fast(tt[k], rare);
      }
      if (rare) {  // one branch per 8 values, rarely taken for ordinary data
        gelu_exact_x8(tt, o);
      }
      __builtin_nontemporal_store(
          o, reinterpret_cast<u32x4_t*>(out + out_off + static_cast<int64_t>(i) * g.C));
    }
  };

  // TPW consecutive position tiles per wave: the next tile's loads are
  // issued before the current one is mapped and stored.
#pragma unroll
  for (int r = 0; r < TPW; ++r) {
    const int ht = ht0 + r;
    if (ht >= g.hw_tiles) break;  // wave-uniform; no barrier follows
    const bool next = r + 1 < TPW && ht + 1 < g.hw_tiles;
    if (r % 2 == 0) {
      if (next) load_tile(ht + 1, vb);
      gelu_store(ht, va);
    } else {
      if (next) load_tile(ht + 1, va);
      gelu_store(ht, vb);
    }
  }
}

// Any shape: one thread per output element, NHWC order (coalesced stores,
// strided loads); the same mapping as the tile kernel, from the table in
// global memory.
__global__ __launch_bounds__(256) void bias_gelu_nchw_to_nhwc_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t N, int64_t C, int64_t HW) {
  const int64_t total = N * C * HW;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       o < total; o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t c = o % C;
    const int64_t p = (o / C) % HW;
    const int64_t img = o / (C * HW);
    const uint32_t tb =
        pack_bf16x2(bf16_to_f32(x[(img * C + c) * HW + p]) + bf16_to_f32(bias[c]), 0.0f) &
        0xffffu;
    out[o] = static_cast<uint16_t>(gelu_bits(tb, kGeluTable));
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
  // Up to kTileMinElems elements the one-element-per-thread kernel is the
  // faster one: a tile wave maps its 4096 values serially (64 per lane), so
  // a launch of few tiles is bound by one wave's instruction stream, not by
  // memory (steady-state: 5.4 against 2.5 us at [3, 320, 8, 10], 5.9
  // against 3.2 us at [4, 128, 28, 28]; 6.7 against 10.8 us at
  // [2, 256, 56, 56], where the tiles win).
  const bool vec = n * c * hw > kTileMinElems && (c % 8 == 0) && (hw % 8 == 0) &&
                   aligned16(x) && aligned16(bias) && aligned16(out);
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
    const int64_t c_groups = (c_tiles + kWavesC - 1) / kWavesC;
    const int64_t hw_groups =
        (hw_tiles + kWavesP * kTilesPerWave - 1) / (kWavesP * kTilesPerWave);
    if (hw_groups <= 65535 && n <= 65535) {
      const dim3 grid(static_cast<unsigned>(c_groups), static_cast<unsigned>(hw_groups),
                      static_cast<unsigned>(n));
      bias_gelu_nchw_to_nhwc_tiles<true, kTilesPerWave>
          <<<grid, dim3(kBlockThreads), 0, stream>>>(x, bias, out, g);
    } else {
      const int64_t blocks = (ntiles + kWavesPerBlock - 1) / kWavesPerBlock;
      bias_gelu_nchw_to_nhwc_tiles<false, 1><<<dim3(static_cast<unsigned>(blocks)),
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
