// Channel bias + GELU(tanh) fused with NCHW -> NHWC (channels-last), bf16.
//
// Semantics (the eager op order of gelu(x + bias) on bf16 tensors):
//   t = bf16(x + bias[c])            (fp32 add, round to nearest even)
//   y = bf16(GELU_tanh(t))
// Because t is a bf16 value there are only 65536 possible inputs to GELU,
// so GELU is a table lookup: kGeluLut[bits(t)] holds the correctly rounded
// bf16 GELU of every bf16 pattern (generated at build time in double
// precision by hip_oracles/gen_tables.py and compiled into the code object).
// That replaces ~17 VALU cycles per element (two quarter-rate
// transcendentals) with ~5 VALU operations and one LDS read, leaving the
// kernel bound by HBM instead of VALU.
//
// Layout: each workgroup (1024 threads, one per CU) first copies the 128 KiB
// table into LDS.  Work unit = one wave64 tile: 64 channels x 64 spatial
// positions of one image.  Lane l owns an 8x8 (channel x position) block:
// cb = l / 8 picks 8 channels, hb = l % 8 picks 8 positions.  It issues 8
// 16-byte loads, one per channel row (the 8 lanes of equal cb read one
// contiguous 128-byte segment of that row), and 8 16-byte stores, one per
// position (the 8 lanes of equal hb write one contiguous 128-byte segment of
// that NHWC row).  The 8x8 transpose happens in registers: the packed bf16
// conversion (v_cvt_pk_bf16_f32) rounds t for two adjacent channels into one
// word, whose halves index the table, and the two looked-up halves form the
// output word -- no LDS staging of the tile and no barrier per tile.
//
// Scheduling: persistent waves walk tiles t, t + W, ... (W = waves in the
// grid), prefetching the next tile into a second register buffer while the
// current one is computed (two buffers used alternately, so no register copy
// forces a wait on the prefetch).  Tiles are numbered channel group fastest,
// then position tile, then image.  Within a workgroup, groups of C/64 waves
// take all channel groups of one position tile, so each group writes whole
// NHWC rows at once, and the groups are spread gridDim.x position tiles
// apart (measured on MI355X: 69.9 us for config 2 against 83 us when a
// workgroup's waves take consecutive tiles).  Loads and stores are
// non-temporal.
// HBM-bound: algorithmic bytes per element = 2 (read) + 2 (write).
#include "hipo_common.h"

namespace hipo {
namespace {

// bf16 bits of GELU_tanh(t) for every bf16 bit pattern t.
__device__ const uint16_t kGeluLut[65536] = {
#include "gelu_tanh_bf16_lut.inc"
};

constexpr int kTileHw = 64;    // positions per wave tile
constexpr int kTileC = 64;     // channels per wave tile
constexpr int kBlockThreads = 1024;
constexpr int kWavesPerBlock = kBlockThreads / kWave;

struct TileGeom {
  int64_t C, HW;
  int c_tiles, hw_tiles, ntiles;  // ntiles < 2^31 (checked on the host)
};

// Base element offsets of lane's 8x8 block in tile t; false if the lane's
// block lies outside the tensor (partial channel / position tiles).  t is
// wave-uniform, so the tile decomposition runs on the scalar unit.
__device__ __forceinline__ bool tile_block(const TileGeom& g, int t, int lane,
                                           int64_t& in_off, int64_t& out_off,
                                           int64_t& c0) {
  t = __builtin_amdgcn_readfirstlane(t);
  const int ct = t % g.c_tiles;
  const int rest = t / g.c_tiles;
  const int ht = rest % g.hw_tiles;
  const int64_t img = rest / g.hw_tiles;
  c0 = static_cast<int64_t>(ct) * kTileC + (lane >> 3) * 8;
  const int64_t p0 = static_cast<int64_t>(ht) * kTileHw + (lane & 7) * 8;
  in_off = (img * g.C + c0) * g.HW + p0;
  out_off = (img * g.HW + p0) * g.C + c0;
  return c0 < g.C && p0 < g.HW;
}

// One lane's share of a tile in flight: 8 channel rows of 8 positions and
// the 8 channel biases, plus where the results go.
struct Block {
  u32x4_t v[8];
  u32x4_t bw;
  int64_t out_off;
  bool ok;
};

// Issue the 9 loads of tile t.  Lanes outside the tensor load from offset 0
// (always valid) and are masked at the store, so the loads are branch-free.
__device__ __forceinline__ void load_block(const TileGeom& g, int t, int lane,
                                           const u32x4_t* __restrict__ x,
                                           const uint16_t* __restrict__ bias, Block& b) {
  int64_t in_off, c0;
  b.ok = tile_block(g, t, lane, in_off, b.out_off, c0);
  if (!b.ok) {
    in_off = 0;
    c0 = 0;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    b.v[j] = __builtin_nontemporal_load(x + ((in_off + j * g.HW) >> 3));
  }
  b.bw = *reinterpret_cast<const u32x4_t*>(bias + c0);
}

// Output word for position i and channels (2k, 2k+1): round t for both
// channels into one word, look both halves up in the table.
__device__ __forceinline__ uint32_t gelu_pair(const uint16_t* lut, const Block& blk,
                                              const float (&b)[8], int i, int k) {
  const uint32_t w0 = blk.v[2 * k][i >> 1];
  const uint32_t w1 = blk.v[2 * k + 1][i >> 1];
  const float x0 = (i & 1) ? bf16hi(w0) : bf16lo(w0);
  const float x1 = (i & 1) ? bf16hi(w1) : bf16lo(w1);
  const uint32_t t = pack_bf16x2(x0 + b[2 * k], x1 + b[2 * k + 1]);
  return static_cast<uint32_t>(lut[t & 0xffffu]) |
         (static_cast<uint32_t>(lut[t >> 16]) << 16);
}

__device__ __forceinline__ void compute_store(const uint16_t* lut, const Block& blk,
                                              u32x4_t* __restrict__ out, int64_t C) {
  float b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = (j & 1) ? bf16hi(blk.bw[j >> 1]) : bf16lo(blk.bw[j >> 1]);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4_t o = {gelu_pair(lut, blk, b, i, 0), gelu_pair(lut, blk, b, i, 1),
                       gelu_pair(lut, blk, b, i, 2), gelu_pair(lut, blk, b, i, 3)};
    if (blk.ok) __builtin_nontemporal_store(o, out + ((blk.out_off + i * C) >> 3));
  }
}

__global__ __launch_bounds__(kBlockThreads) void bias_gelu_nchw_to_nhwc_tiles(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, TileGeom g) {
  __shared__ u32x4_t lut_words[65536 * 2 / 16];
  {
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(kGeluLut);
#pragma unroll
    for (int k = 0; k < 65536 * 2 / 16 / kBlockThreads; ++k) {
      lut_words[threadIdx.x + k * kBlockThreads] = src[threadIdx.x + k * kBlockThreads];
    }
  }
  __syncthreads();
  const uint16_t* lut = reinterpret_cast<const uint16_t*>(lut_words);

  const int lane = threadIdx.x & (kWave - 1);
  const int nwaves = static_cast<int>(gridDim.x) * kWavesPerBlock;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  int t;
  if (kWavesPerBlock % g.c_tiles == 0) {
    // Groups of c_tiles waves take all channel tiles of one position tile
    // (so a group writes whole NHWC rows together); the groups of a
    // workgroup are spread gridDim.x position tiles apart.
    const int group = w / g.c_tiles;
    t = (static_cast<int>(blockIdx.x) + group * static_cast<int>(gridDim.x)) * g.c_tiles +
        w % g.c_tiles;
  } else {
    t = static_cast<int>(blockIdx.x) + w * static_cast<int>(gridDim.x);
  }
  if (t >= g.ntiles) return;  // wave-uniform; after the only barrier
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x);
  u32x4_t* ov = reinterpret_cast<u32x4_t*>(out);

  // Software pipeline with two register buffers used alternately: the next
  // tile's loads are in flight while the current tile is computed, and no
  // register copy (which would wait for those loads) separates iterations.
  Block a, b;
  load_block(g, t, lane, xv, bias, a);
  while (true) {
    if (t + nwaves >= g.ntiles) {
      compute_store(lut, a, ov, g.C);
      break;
    }
    load_block(g, t + nwaves, lane, xv, bias, b);
    compute_store(lut, a, ov, g.C);
    t += nwaves;
    if (t + nwaves >= g.ntiles) {
      compute_store(lut, b, ov, g.C);
      break;
    }
    load_block(g, t + nwaves, lane, xv, bias, a);
    compute_store(lut, b, ov, g.C);
    t += nwaves;
  }
}

// Any shape: one thread per output element, NHWC order (coalesced stores,
// strided loads), table read from global memory.
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
    out[o] = kGeluLut[pack_bf16x2(t, 0.0f) & 0xffffu];
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
    HIPO_REQUIRE(ntiles < (int64_t{1} << 31) - (int64_t{1} << 20),
                 "bias_gelu: %lld tiles exceed the 32-bit tile index",
                 (long long)ntiles);
    TileGeom g;
    g.C = c;
    g.HW = hw;
    g.c_tiles = static_cast<int>(c_tiles);
    g.hw_tiles = static_cast<int>(hw_tiles);
    g.ntiles = static_cast<int>(ntiles);
    const DeviceInfo* dev = device_info();
    HIPO_REQUIRE(dev != nullptr, "bias_gelu: no current HIP device");
    // One 1024-thread workgroup per CU (the table takes 128 KiB of LDS).
    int64_t blocks = dev->cu_count;
    const int64_t need = (ntiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > need) blocks = need;
    bias_gelu_nchw_to_nhwc_tiles<<<dim3(static_cast<unsigned>(blocks)),
                                   dim3(kBlockThreads), 0, stream>>>(x, bias, out, g);
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
