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
  // Eight loads per lane in flight before any add (one at a time, every
  // iteration waited a full memory latency); the adds keep the order
  // i = lane, lane + 64, ... and skip what lies past the row, so the sum is
  // the same as a one-by-one loop's.
  constexpr int kBatch = 8;
  float acc = 0.f;
  for (int64_t i0 = lane; i0 < cols; i0 += int64_t{kWave} * kBatch) {
    float v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t i = i0 + int64_t{k} * kWave;
      v[k] = i < cols ? p[i] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (i0 + int64_t{k} * kWave < cols) acc += v[k];
  }
  const float s = wave_sum(acc);
  if (lane == 0) out[row] = s / static_cast<float>(cols);
}


// bf16 rows, fp32 accumulation, optional ReLU (NaN kept):
//   out[r] = bf16(sum_j act(x[r, j]) / cols)   (one rounding, nearest even).
// Short rows (cols <= 512, contiguous, 16-byte aligned x): each wave takes 8
// consecutive rows -- 16 * cols bytes, a whole number of 16-byte vectors
// whatever cols is, so the input is read as one flat stream of non-temporal
// vector loads (the SqueezeNet rows are 169 elements, 338 bytes, not
// vector-aligned one by one).  The wave stages its 8 rows in LDS; then 8
// lanes per row sum every 8th element in order and combine in a fixed
// DPP butterfly.  Longer rows: one wave per row.
constexpr int kBf16RowsPerWave = 8;
constexpr int kBf16ShortCols = 512;
constexpr int kBf16Waves = 4;

template <bool RELU>
__device__ __forceinline__ float act_relu(float v) {
  return RELU ? __builtin_elementwise_maximum(v, 0.0f) : v;
}

__device__ __forceinline__ uint16_t round_to_bf16(float v) {
  return static_cast<uint16_t>(pack_bf16x2(v, 0.0f) & 0xffffu);
}

template <bool RELU, int VPL>
__global__ __launch_bounds__(kBf16Waves * kWave) void row_mean_bf16_short(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ out, int64_t rows, int cols) {
  __shared__ __align__(16) uint16_t stage[kBf16Waves][kBf16RowsPerWave * kBf16ShortCols];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kBf16Waves + wave) * kBf16RowsPerWave;
  const int64_t nrows = rows - row0 < kBf16RowsPerWave ? rows - row0 : kBf16RowsPerWave;
  uint16_t* lds = stage[wave];
  if (nrows > 0) {
    // The wave's rows: `cols` vectors of 16 bytes when all 8 rows exist;
    // the last group may end inside a vector, whose elements move singly.
    const int64_t elems = nrows * cols;
    const int whole = static_cast<int>(elems / 8);
    const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x + row0 * cols);
    if (whole > 0) {  // wave-uniform
      // Loads without a branch (slots past the end reload the last vector),
      // so all of them are in flight before the first is used.
      u32x4_t v[VPL];
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const int i = lane + k * kWave;
        v[k] = __builtin_nontemporal_load(xv + (i < whole ? i : whole - 1));
      }
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const int i = lane + k * kWave;
        if (i < whole) reinterpret_cast<u32x4_t*>(lds)[i] = v[k];
      }
    }
    const int rest = static_cast<int>(elems - int64_t{whole} * 8);
    if (lane < rest) lds[whole * 8 + lane] = x[row0 * cols + whole * 8 + lane];
  }
  __syncthreads();
  if (nrows <= 0) return;
  const int r = lane >> 3;   // row of the group
  const int k = lane & 7;    // this lane's residue class
  float s = 0.0f;
  if (r < nrows) {
    const uint16_t* p = lds + r * cols;
    for (int j = k; j < cols; j += 8) s += act_relu<RELU>(bf16_to_f32(p[j]));
  }
  s = sum8(s);
  if (k == 0 && r < nrows) out[row0 + r] = round_to_bf16(s / static_cast<float>(cols));
}

template <bool RELU, bool VEC>
__global__ __launch_bounds__(256) void row_mean_bf16_long(const uint16_t* __restrict__ x,
                                                          uint16_t* __restrict__ out,
                                                          int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform; no barrier follows
  const uint16_t* p = x + row * cols;
  float acc = 0.0f;
  if constexpr (VEC) {
    const u32x4_t* pv = reinterpret_cast<const u32x4_t*>(p);
    for (int64_t i = lane; i < cols / 8; i += kWave) {
      const u32x4_t w = __builtin_nontemporal_load(pv + i);
      float t = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        t += act_relu<RELU>(bf16lo(w[q])) + act_relu<RELU>(bf16hi(w[q]));
      acc += t;
    }
  } else {
    for (int64_t i = lane; i < cols; i += kWave) acc += act_relu<RELU>(bf16_to_f32(p[i]));
  }
  const float s = wave_sum(acc);
  if (lane == 0) out[row] = round_to_bf16(s / static_cast<float>(cols));
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

extern "C" int hipo_row_mean_bf16(const uint16_t* x, uint16_t* out, int64_t rows,
                                  int64_t cols, int relu, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "row_mean_bf16: negative size");
  if (rows == 0) return 0;
  HIPO_REQUIRE(cols > 0, "row_mean_bf16: mean over zero elements");
  HIPO_REQUIRE(x != nullptr && out != nullptr, "row_mean_bf16: null pointer");
  const bool act = relu != 0;
  if (cols <= kBf16ShortCols && aligned16(x)) {
    const int64_t groups = (rows + kBf16RowsPerWave - 1) / kBf16RowsPerWave;
    const int64_t blocks = (groups + kBf16Waves - 1) / kBf16Waves;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "row_mean_bf16: too many rows");
    const dim3 grid(static_cast<unsigned>(blocks)), block(kBf16Waves * kWave);
    const int c = static_cast<int>(cols);
    // cols vectors of 16 bytes per wave: ceil(cols / 64) per lane.
#define HIPO_RMB(V_)                                                                    \
  (act ? row_mean_bf16_short<true, V_><<<grid, block, 0, stream>>>(x, out, rows, c)     \
       : row_mean_bf16_short<false, V_><<<grid, block, 0, stream>>>(x, out, rows, c))
    if (cols <= 2 * kWave) {
      HIPO_RMB(2);
    } else if (cols <= 4 * kWave) {
      HIPO_RMB(4);
    } else {
      HIPO_RMB(8);
    }
#undef HIPO_RMB
  } else {
    const bool vec = cols % 8 == 0 && aligned16(x);
    const int64_t blocks = (rows + 3) / 4;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "row_mean_bf16: too many rows");
    const dim3 grid(static_cast<unsigned>(blocks)), block(256);
    if (vec) {
      if (act) row_mean_bf16_long<true, true><<<grid, block, 0, stream>>>(x, out, rows, cols);
      else row_mean_bf16_long<false, true><<<grid, block, 0, stream>>>(x, out, rows, cols);
    } else {
      if (act) row_mean_bf16_long<true, false><<<grid, block, 0, stream>>>(x, out, rows, cols);
      else row_mean_bf16_long<false, false><<<grid, block, 0, stream>>>(x, out, rows, cols);
    }
  }
  return check_launch("row_mean_bf16");
}
