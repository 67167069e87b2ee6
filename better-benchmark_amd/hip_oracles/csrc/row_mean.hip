// Row mean, fp32: out[r] = sum(x[r, :]) / cols.
//
// Several waves per row.  A workgroup holds `rows_per_block` rows of
// `waves_per_row` waves each (at most 8 waves).  Lane l of wave w of a row
// reads float4 index  (it * U + u) * W * 64 + w * 64 + l  (W = waves per
// row), so every load instruction of a wave covers 1 KiB of contiguous row
// and the W waves of a row sweep it together.  Each lane keeps U
// non-temporal 16-byte loads in flight, accumulates in fp32, the wave
// reduces with DPP, and the W wave sums are added in LDS in a fixed order.
//
// Measured on MI355X for [8192, 4096]: 8 waves x 2 float4 per lane reads at
// 81 % of 8 TB/s; one wave per row with 16 float4 per lane reaches 67 %
// (73 % with non-temporal loads) -- smaller per-wave footprints keep the
// in-flight address window compact.
// HBM-bound: algorithmic bytes per row = 4*cols (read) + 4 (write).
#include <algorithm>

#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kMaxWaves = 8;  // per workgroup
constexpr int kMaxThreads = kMaxWaves * kWave;

// WT > 0: waves per row (and rows per workgroup, kMaxWaves / WT) fixed at
// compile time; WT = 0: both from the arguments.
template <int U, int WT>
__global__ __launch_bounds__(kMaxThreads) void row_mean_f32_vec4(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows,
    int64_t cols, int64_t row_stride, int w_arg, int rpb_arg) {
  const int waves_per_row = WT > 0 ? WT : w_arg;
  const int rows_per_block = WT > 0 ? kMaxWaves / WT : rpb_arg;
  __shared__ float part[kMaxWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int w = wave % waves_per_row;
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * rows_per_block + wave / waves_per_row;
  // Waves past the last row still take part in the barrier; they read the
  // last row and write nothing.
  const bool valid = row < rows;
  const f32x4_t* p =
      reinterpret_cast<const f32x4_t*>(x + (valid ? row : rows - 1) * row_stride);
  const int64_t nvec = cols >> 2;
  const int64_t step = static_cast<int64_t>(waves_per_row) * kWave;

  const int64_t sweeps = (nvec + step * U - 1) / (step * U);

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t it = 0; it < sweeps; ++it) {
    const int64_t base = it * step * U + w * kWave + lane;
    f32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // Out-of-row slots load the row's last float4 (in bounds, no branch
      // around the load) and are zeroed.
      const int64_t i = base + u * step;
      v[u] = __builtin_nontemporal_load(p + (i < nvec ? i : nvec - 1));
      if (i >= nvec) v[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u];
  }
  float s = wave_sum((acc.x + acc.y) + (acc.z + acc.w));
  if (waves_per_row > 1) {
    if (lane == 0) part[wave] = s;
    __syncthreads();
    const int first = wave - w;
    s = part[first];
    for (int k = 1; k < waves_per_row; ++k) s += part[first + k];
  }
  if (valid && w == 0 && lane == 0) out[row] = s / static_cast<float>(cols);
}

// Any alignment / any cols: scalar loads, one wave per row.
__global__ __launch_bounds__(256) void row_mean_f32_scalar(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows,
    int64_t cols, int64_t row_stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* p = x + row * row_stride;
  float acc = 0.f;
  for (int64_t i = lane; i < cols; i += kWave) acc += p[i];
  const float s = wave_sum(acc);
  if (lane == 0) out[row] = s / static_cast<float>(cols);
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_row_mean_f32(const float* x, float* out, int64_t rows,
                                 int64_t cols, int64_t row_stride,
                                 hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "row_mean: negative size");
  HIPO_REQUIRE(row_stride >= cols, "row_mean: row_stride %lld < cols %lld",
               (long long)row_stride, (long long)cols);
  if (rows == 0) return 0;
  HIPO_REQUIRE(x != nullptr && out != nullptr, "row_mean: null pointer");
  const bool vec = cols >= 4 && (cols % 4 == 0) && (row_stride % 4 == 0) &&
                   aligned16(x);
  if (vec) {
    // About 2 KiB per wave: W = ceil(nvec / 128) waves per row (at most 8),
    // U = float4 per lane per sweep.
    const int64_t nvec = cols / 4;
    const int waves = static_cast<int>(
        std::min<int64_t>(kMaxWaves, (nvec + 2 * kWave - 1) / (2 * kWave)));
    const int64_t per_lane = (nvec + int64_t{waves} * kWave - 1) / (int64_t{waves} * kWave);
    const int rpb = kMaxWaves / waves;
    const int64_t blocks = (rows + rpb - 1) / rpb;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "row_mean: too many rows");
    const dim3 grid(static_cast<unsigned>(blocks)), block(waves * rpb * kWave);
#define HIPO_MEAN(U_, W_)                                                            \
  row_mean_f32_vec4<U_, W_><<<grid, block, 0, stream>>>(x, out, rows, cols, row_stride, \
                                                        waves, rpb)
#define HIPO_MEAN_W(U_)                                  \
  switch (waves) {                                       \
    case 1: HIPO_MEAN(U_, 1); break;                     \
    case 2: HIPO_MEAN(U_, 2); break;                     \
    case 4: HIPO_MEAN(U_, 4); break;                     \
    case 8: HIPO_MEAN(U_, 8); break;                     \
    default: HIPO_MEAN(U_, 0); break;                    \
  }
    if (per_lane <= 1) {
      HIPO_MEAN_W(1);
    } else if (per_lane <= 2) {
      HIPO_MEAN_W(2);
    } else {
      HIPO_MEAN_W(4);
    }
#undef HIPO_MEAN_W
#undef HIPO_MEAN
  } else {
    const int64_t blocks = (rows + 3) / 4;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "row_mean: too many rows");
    row_mean_f32_scalar<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                          stream>>>(x, out, rows, cols, row_stride);
  }
  return check_launch("row_mean_f32");
}
