// Row mean, fp32: out[r] = sum(x[r, :]) / cols.
//
// One wave64 per row, four rows per 256-thread workgroup.  The fast path
// reads each row with 16-byte loads (lane-interleaved, so every load
// instruction covers 1 KiB of contiguous row), keeps UNROLL loads in flight
// per lane, accumulates in fp32 and finishes with a DPP wave reduction.
// HBM-bound: algorithmic bytes per row = 4*cols (read) + 4 (write).
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kUnroll = 16;

__global__ __launch_bounds__(256) void row_mean_f32_vec4(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows,
    int64_t cols, int64_t row_stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // row is wave-uniform: whole waves leave
  const float4* p = reinterpret_cast<const float4*>(x + row * row_stride);
  const int64_t nvec = cols >> 2;

  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t base = 0; base < nvec; base += kWave * kUnroll) {
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * kWave + lane;
      v[u] = i < nvec ? p[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc.x += v[u].x;
      acc.y += v[u].y;
      acc.z += v[u].z;
      acc.w += v[u].w;
    }
  }
  const float s = wave_sum((acc.x + acc.y) + (acc.z + acc.w));
  if (lane == 0) out[row] = s / static_cast<float>(cols);
}

// Any alignment / any cols: scalar loads, same wave-per-row structure.
__global__ __launch_bounds__(256) void row_mean_f32_scalar(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows,
    int64_t cols, int64_t row_stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
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
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  HIPO_REQUIRE(blocks <= 0x7fffffff, "row_mean: too many rows");
  const bool vec = (cols % 4 == 0) && (row_stride % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  if (vec) {
    row_mean_f32_vec4<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                        stream>>>(x, out, rows, cols, row_stride);
  } else {
    row_mean_f32_scalar<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                          stream>>>(x, out, rows, cols, row_stride);
  }
  return check_launch("row_mean_f32");
}
