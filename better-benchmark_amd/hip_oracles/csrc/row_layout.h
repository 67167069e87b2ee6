// Work layout shared by the bf16 row kernels (LayerNorm, RMSNorm, softmax).
//
// A workgroup holds `rows_per_block` rows of `waves_per_row` waves each (at
// most kRowMaxWaves waves).  A row of `cols` bf16 values is cut into groups
// of 8 (16 bytes); lane l of wave w of a row owns groups
//     g = (u * W + w) * 64 + l,   u = 0 .. U-1   (W = waves per row)
// so each 16-byte access instruction of a wave covers 1 KiB of contiguous
// row and the W waves sweep the row together.  The whole row stays in
// registers between its statistics and its output.
//
// Waves whose row is past the last one still run (they take part in the
// workgroup barrier): they read the last row and store nothing.  Groups
// past the end of the row load the row's last group (the load stays in
// bounds and needs no branch, which would make the compiler wait on each
// load separately) and are zeroed.
//
// Shape: the host picks W so that a wave holds about 2 KiB of each streamed
// tensor (2 groups per lane) and packs rows so a workgroup has 8 waves.
// Measured on MI355X, same process, interleaved: RMSNorm / LayerNorm
// [16384, 4096] at 4 waves x 2 groups, 2 rows per workgroup: 74.6 / 75.0 %
// of 8 TB/s, against 73.0 / 73.0 % at 2 waves x 4 groups (2 rows), 67-72 %
// at 8 waves x 1 group, 71 % at 1 wave x 8 groups; softmax [384*1024, 1024]
// at 1 wave x 2 groups, 8 rows per workgroup: 77.3 %, against 74.7 % at 4
// rows and 68-70 % at 2 waves x 1 group.  One wave per row with 8 groups
// per lane and cached accesses (the first version): 59-64 %.
#pragma once

#include <algorithm>

#include "hipo_common.h"

namespace hipo {

constexpr int kRowMaxWaves = 8;
constexpr int kRowMaxThreads = kRowMaxWaves * kWave;
constexpr int kRowGroup = 8;                     // bf16 per 16-byte group
constexpr int kRowSweep = kRowGroup * kWave;     // bf16 per wave per sweep

struct RowPlace {
  int lane;
  int wave;     // in the workgroup
  int w;        // in the row
  int64_t row;  // clamped to the last row
  bool valid;   // row < rows
};

__device__ __forceinline__ RowPlace row_place(int waves_per_row,
                                              int rows_per_block,
                                              int64_t rows) {
  RowPlace p;
  p.lane = threadIdx.x & (kWave - 1);
  p.wave = threadIdx.x >> 6;
  p.w = p.wave % waves_per_row;
  const int64_t r =
      static_cast<int64_t>(blockIdx.x) * rows_per_block + p.wave / waves_per_row;
  p.valid = r < rows;
  p.row = p.valid ? r : rows - 1;
  return p;
}

// First column of the lane's u-th group.
__device__ __forceinline__ int64_t row_group_col(int u, int waves_per_row,
                                                 const RowPlace& p) {
  return (static_cast<int64_t>(u * waves_per_row + p.w) * kWave + p.lane) *
         kRowGroup;
}

// Valid values in wave w's groups of a row of `cols` (cols % 8 == 0).
__device__ __forceinline__ int row_wave_count(int U, int waves_per_row,
                                              const RowPlace& p, int64_t cols) {
  int n = 0;
  for (int u = 0; u < U; ++u) {
    const int64_t first = static_cast<int64_t>(u * waves_per_row + p.w) * kRowSweep;
    const int64_t left = cols - first;
    n += static_cast<int>(left <= 0 ? 0 : (left < kRowSweep ? left : kRowSweep));
  }
  return n;
}

// 8 bf16 of `row` at `col` (non-temporal), or zeros past the row end.
__device__ __forceinline__ u32x4_t row_load_stream(const uint16_t* row,
                                                   int64_t col, int64_t cols) {
  const int64_t c = col < cols ? col : cols - kRowGroup;
  const u32x4_t v =
      __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row + c));
  return col < cols ? v : u32x4_t{0u, 0u, 0u, 0u};
}

// 8 bf16 of a vector that every row re-reads (gamma, beta, mask rows):
// cached load, zeros past the end.
__device__ __forceinline__ u32x4_t row_load_cached(const uint16_t* v, int64_t col,
                                                   int64_t cols) {
  const int64_t c = col < cols ? col : cols - kRowGroup;
  const u32x4_t r = *reinterpret_cast<const u32x4_t*>(v + c);
  return col < cols ? r : u32x4_t{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ void row_store_stream(uint16_t* row, int64_t col,
                                                 u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(row + col));
}

// Short rows (cols <= 512): a row owns L = 2^j consecutive lanes (L groups
// of 8 bf16), so one 16-byte access instruction of a wave covers 64 / L
// rows.  seg_sum / seg_max reduce within each aligned segment of L lanes
// (DPP quad swaps, half-row and row mirrors; across 16-lane rows the row
// results read back with v_readlane, no LDS round trip); every lane of a
// segment receives the same value, and the order of the additions is fixed
// (the same additions as lane-xor shuffles of 16 and 32 would make, so the
// same bits).  All 64 lanes must be active.  (Readlanes instead of the two
// shuffles: [16384, 768] / [16384, 1024] LayerNorm 14.4 -> 14.1 / 18.3 ->
// 18.0 us back to back; L = 32 rows unchanged.)
constexpr int kDppRowMirror = 0x140;  // lane i <- 15 - i within a row

__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

template <int L>
__device__ __forceinline__ float seg_sum(float v) {
  if constexpr (L >= 2) v += dpp<kDppQuadXor1>(v);
  if constexpr (L >= 4) v += dpp<kDppQuadXor2>(v);
  if constexpr (L >= 8) v += dpp<kDppRowHalfMirror>(v);
  if constexpr (L >= 16) v += dpp<kDppRowMirror>(v);
  if constexpr (L >= 32) {
    const float a = lane_value(v, 0), b = lane_value(v, 16);
    const float c = lane_value(v, 32), d = lane_value(v, 48);
    if constexpr (L >= 64) {
      v = (a + b) + (c + d);
    } else {
      v = __lane_id() < 32 ? a + b : c + d;
    }
  }
  return v;
}

template <int L>
__device__ __forceinline__ float seg_max(float v) {
  if constexpr (L >= 2) v = fmaxf(v, dpp<kDppQuadXor1>(v));
  if constexpr (L >= 4) v = fmaxf(v, dpp<kDppQuadXor2>(v));
  if constexpr (L >= 8) v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
  if constexpr (L >= 16) v = fmaxf(v, dpp<kDppRowMirror>(v));
  if constexpr (L >= 32) {
    const float a = lane_value(v, 0), b = lane_value(v, 16);
    const float c = lane_value(v, 32), d = lane_value(v, 48);
    if constexpr (L >= 64) {
      v = fmaxf(fmaxf(a, b), fmaxf(c, d));
    } else {
      v = __lane_id() < 32 ? fmaxf(a, b) : fmaxf(c, d);
    }
  }
  return v;
}

// Lanes per row for a short row (0: not short).
inline int short_row_lanes(int64_t cols) {
  if (cols <= 0 || cols > kRowSweep) return 0;
  int L = 1;
  while (L * kRowGroup < cols) L *= 2;
  return L;
}

// Host side: waves per row, groups per lane, rows per workgroup for a row of
// `cols` bf16 values (cols % 8 == 0).  Groups per lane are rounded up to a
// power of two (the kernels are instantiated for 1, 2, 4, 8); returns false
// if the row does not fit in registers (cols > 8 waves x 8 groups x 512).
struct RowPlan {
  int waves_per_row;
  int groups;  // U
  int rows_per_block;
  int threads() const { return waves_per_row * rows_per_block * kWave; }
};

// Launch LAUNCH(U, WT) for a row plan.  WT > 0 fixes the waves per row
// (and so the rows per workgroup, kRowMaxWaves / WT) at compile time for
// the (W, U) pairs row_plan produces with W a power of two; WT = 0 takes
// both from the kernel arguments.  Measured on MI355X (RMSNorm [16384,
// 4096], W = 4, U = 2): 45.0 us with runtime W, 43.8 us with WT = 4 -- the
// constant folds the row placement and the fixed-order LDS combine of the
// per-row sums.
#define HIPO_ROW_DISPATCH(plan, LAUNCH)                            \
  do {                                                             \
    const int w_ = (plan).waves_per_row, u_ = (plan).groups;       \
    if (w_ == 1 && u_ == 1) {                                      \
      LAUNCH(1, 1);                                                \
    } else if (w_ == 1 && u_ == 2) {                               \
      LAUNCH(2, 1);                                                \
    } else if (w_ == 2 && u_ == 2) {                               \
      LAUNCH(2, 2);                                                \
    } else if (w_ == 4 && u_ == 2) {                               \
      LAUNCH(2, 4);                                                \
    } else if (w_ == 8 && u_ == 2) {                               \
      LAUNCH(2, 8);                                                \
    } else if (w_ == 8 && u_ == 4) {                               \
      LAUNCH(4, 8);                                                \
    } else if (w_ == 8 && u_ == 8) {                               \
      LAUNCH(8, 8);                                                \
    } else if (u_ == 1) {                                          \
      LAUNCH(1, 0);                                                \
    } else if (u_ == 2) {                                          \
      LAUNCH(2, 0);                                                \
    } else if (u_ == 4) {                                          \
      LAUNCH(4, 0);                                                \
    } else {                                                       \
      LAUNCH(8, 0);                                                \
    }                                                              \
  } while (0)

inline bool row_plan(int64_t cols, RowPlan& plan) {
  // About 2 groups (2 KiB) per wave of each streamed tensor, 8 waves per
  // workgroup.  (RMSNorm at [16384, 4096], back to back: 4 waves per row x
  // 2 groups 45.2-45.4 us, 2 x 4 46.9-47.3, 1 x 8 50.0-50.2.)  (One group per wave for the two streams of LayerNorm was
  // faster with outputs reused across launches, slower in the steady loop
  // where every step writes fresh output buffers: 91.7-92.3 against
  // 89.7-89.9 us at [16384, 4096].)  (LayerNorm rows of 2560: 5 waves x 1
  // group, no idle lanes, against this plan's 3 x 2: y only [4096, 2560]
  // 15.5 against 14.3 us and [2048, 2560] 9.4 against 7.5 back to back; h
  // and y [4096, 2560] 17.3 against 18.2.)
  const int64_t per_wave = 2 * kRowSweep;
  const int64_t w = std::min<int64_t>(kRowMaxWaves, (cols + per_wave - 1) / per_wave);
  plan.waves_per_row = static_cast<int>(std::max<int64_t>(1, w));
  const int64_t sweep = int64_t{plan.waves_per_row} * kRowSweep;
  const int64_t u = (cols + sweep - 1) / sweep;
  if (u > 8) return false;
  plan.groups = u <= 1 ? 1 : u <= 2 ? 2 : u <= 4 ? 4 : 8;
  plan.rows_per_block = std::max(1, kRowMaxWaves / plan.waves_per_row);
  return true;
}

}  // namespace hipo
