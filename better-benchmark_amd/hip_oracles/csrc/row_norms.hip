// Row normalisations over the last dim, bf16 in / bf16 out, fp32 statistics:
//   residual-add LayerNorm  (outputs h, y, mean, rstd)
//   RMSNorm                 (outputs y, rstd)
//
// One wave64 per row, four rows per 256-thread workgroup.  The row stays in
// registers between the statistics and the normalisation: lane l owns
// elements [c*512 + 8l, +8) of chunk c, moved with one 16-byte access per
// chunk per tensor.  LayerNorm statistics are two-pass over the registers
// (mean, then sum of squared deviations), reduced with DPP; gamma/beta rows
// are re-read by every row and stay cache-resident.
//
// HBM-bound.  Algorithmic bytes per row (cols = C):
//   residual LayerNorm: 2C (x) + 2C (residual) + 2C (h) + 2C (y) + 8
//   RMSNorm:            2C (x) + 2C (y) + 4
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kChunk = 8 * kWave;

template <int NCH>
__global__ __launch_bounds__(256) void residual_layernorm_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    uint16_t* __restrict__ h, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t rows,
    int64_t cols, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int64_t base = row * cols;

  uint4 xv[NCH], rv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < cols) {
      xv[c] = *reinterpret_cast<const uint4*>(x + base + col);
      rv[c] = *reinterpret_cast<const uint4*>(res + base + col);
    } else {
      xv[c] = make_uint4(0u, 0u, 0u, 0u);
      rv[c] = make_uint4(0u, 0u, 0u, 0u);
    }
  }

  // h = bf16(x + residual); statistics use the bf16-rounded h.
  uint4 hv[NCH];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const uint32_t xw[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    const uint32_t rw[4] = {rv[c].x, rv[c].y, rv[c].z, rv[c].w};
    uint32_t hw[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      hw[d] = pack_bf16x2(bf16lo(xw[d]) + bf16lo(rw[d]),
                          bf16hi(xw[d]) + bf16hi(rw[d]));
      sum += bf16lo(hw[d]) + bf16hi(hw[d]);
    }
    hv[c] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < cols) *reinterpret_cast<uint4*>(h + base + col) = hv[c];
  }
  const float fcols = static_cast<float>(cols);
  const float mean = wave_sum(sum) / fcols;

  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < cols) {
      const uint32_t w[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float a = bf16lo(w[d]) - mean;
        const float b = bf16hi(w[d]) - mean;
        sq = __builtin_fmaf(a, a, sq);
        sq = __builtin_fmaf(b, b, sq);
      }
    }
  }
  const float var = wave_sum(sq) / fcols;
  const float rstd = 1.0f / __builtin_sqrtf(var + eps);
  const float shift = -mean * rstd;

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < cols) {
      const uint4 gv = *reinterpret_cast<const uint4*>(gamma + col);
      const uint4 bv = *reinterpret_cast<const uint4*>(beta + col);
      const uint32_t w[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
      const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
      uint32_t o[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float n0 = __builtin_fmaf(bf16lo(w[d]), rstd, shift);
        const float n1 = __builtin_fmaf(bf16hi(w[d]), rstd, shift);
        o[d] = pack_bf16x2(__builtin_fmaf(n0, bf16lo(gw[d]), bf16lo(bw[d])),
                           __builtin_fmaf(n1, bf16hi(gw[d]), bf16hi(bw[d])));
      }
      *reinterpret_cast<uint4*>(y + base + col) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  if (lane == 0) {
    mean_out[row] = mean;
    rstd_out[row] = rstd;
  }
}

template <int NCH>
__global__ __launch_bounds__(256) void rmsnorm_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    uint16_t* __restrict__ y, float* __restrict__ rstd_out, int64_t rows,
    int64_t cols, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;

  uint4 xv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    xv[c] = col < cols ? *reinterpret_cast<const uint4*>(x + base + col)
                       : make_uint4(0u, 0u, 0u, 0u);
  }
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const uint32_t w[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = bf16lo(w[d]);
      const float b = bf16hi(w[d]);
      sq = __builtin_fmaf(a, a, sq);
      sq = __builtin_fmaf(b, b, sq);
    }
  }
  const float ms = wave_sum(sq) / static_cast<float>(cols);
  const float rstd = 1.0f / __builtin_sqrtf(ms + eps);

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < cols) {
      const uint4 gv = *reinterpret_cast<const uint4*>(gamma + col);
      const uint32_t w[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
      uint32_t o[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        o[d] = pack_bf16x2((bf16lo(w[d]) * rstd) * bf16lo(gw[d]),
                           (bf16hi(w[d]) * rstd) * bf16hi(gw[d]));
      }
      *reinterpret_cast<uint4*>(y + base + col) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  if (lane == 0) rstd_out[row] = rstd;
}

// Any cols / alignment: one wave per row, scalar accesses, row re-read from
// memory for each pass.
__global__ __launch_bounds__(256) void residual_layernorm_rows_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    uint16_t* __restrict__ h, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t rows,
    int64_t cols, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float sum = 0.f;
  for (int64_t j = lane; j < cols; j += kWave) {
    const float hv = round_bf16(bf16_to_f32(x[base + j]) + bf16_to_f32(res[base + j]));
    h[base + j] = static_cast<uint16_t>(pack_bf16x2(hv, 0.f) & 0xffffu);
    sum += hv;
  }
  const float mean = wave_sum(sum) / static_cast<float>(cols);
  float sq = 0.f;
  for (int64_t j = lane; j < cols; j += kWave) {
    const float a =
        round_bf16(bf16_to_f32(x[base + j]) + bf16_to_f32(res[base + j])) - mean;
    sq = __builtin_fmaf(a, a, sq);
  }
  const float rstd =
      1.0f / __builtin_sqrtf(wave_sum(sq) / static_cast<float>(cols) + eps);
  const float shift = -mean * rstd;
  for (int64_t j = lane; j < cols; j += kWave) {
    const float hv = round_bf16(bf16_to_f32(x[base + j]) + bf16_to_f32(res[base + j]));
    const float v = __builtin_fmaf(__builtin_fmaf(hv, rstd, shift),
                                   bf16_to_f32(gamma[j]), bf16_to_f32(beta[j]));
    y[base + j] = static_cast<uint16_t>(pack_bf16x2(v, 0.f) & 0xffffu);
  }
  if (lane == 0) {
    mean_out[row] = mean;
    rstd_out[row] = rstd;
  }
}

__global__ __launch_bounds__(256) void rmsnorm_rows_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
    uint16_t* __restrict__ y, float* __restrict__ rstd_out, int64_t rows,
    int64_t cols, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float sq = 0.f;
  for (int64_t j = lane; j < cols; j += kWave) {
    const float a = bf16_to_f32(x[base + j]);
    sq = __builtin_fmaf(a, a, sq);
  }
  const float rstd =
      1.0f / __builtin_sqrtf(wave_sum(sq) / static_cast<float>(cols) + eps);
  for (int64_t j = lane; j < cols; j += kWave) {
    const float v = (bf16_to_f32(x[base + j]) * rstd) * bf16_to_f32(gamma[j]);
    y[base + j] = static_cast<uint16_t>(pack_bf16x2(v, 0.f) & 0xffffu);
  }
  if (lane == 0) rstd_out[row] = rstd;
}

}  // namespace
}  // namespace hipo

#define HIPO_NCH_SWITCH(nch, KERNEL, grid, stream, ...)                      \
  switch (nch) {                                                             \
    case 1: KERNEL<1><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    case 2: KERNEL<2><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    case 3: KERNEL<3><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    case 4: KERNEL<4><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    case 5: KERNEL<5><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    case 6: KERNEL<6><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    case 7: KERNEL<7><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;   \
    default: KERNEL<8><<<grid, dim3(256), 0, stream>>>(__VA_ARGS__); break;  \
  }

extern "C" int hipo_residual_layernorm_bf16(
    const uint16_t* x, const uint16_t* residual, const uint16_t* gamma,
    const uint16_t* beta, uint16_t* h, uint16_t* y, float* mean, float* rstd,
    int64_t rows, int64_t cols, float eps, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "residual_layernorm: negative size");
  if (rows == 0) return 0;
  HIPO_REQUIRE(cols > 0, "residual_layernorm: cols must be > 0");
  HIPO_REQUIRE(x && residual && gamma && beta && h && y && mean && rstd,
               "residual_layernorm: null pointer");
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  HIPO_REQUIRE(blocks <= 0x7fffffff, "residual_layernorm: too many rows");
  const dim3 grid(static_cast<unsigned>(blocks));
  const int64_t nch = (cols + kChunk - 1) / kChunk;
  const bool vec = cols % 8 == 0 && nch <= 8 && aligned16(x) &&
                   aligned16(residual) && aligned16(gamma) && aligned16(beta) &&
                   aligned16(h) && aligned16(y);
  if (vec) {
    HIPO_NCH_SWITCH(nch, residual_layernorm_rows, grid, stream, x, residual,
                    gamma, beta, h, y, mean, rstd, rows, cols, eps);
  } else {
    residual_layernorm_rows_scalar<<<grid, dim3(256), 0, stream>>>(
        x, residual, gamma, beta, h, y, mean, rstd, rows, cols, eps);
  }
  return check_launch("residual_layernorm_bf16");
}

extern "C" int hipo_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma,
                                 uint16_t* y, float* rstd, int64_t rows,
                                 int64_t cols, float eps, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "rmsnorm: negative size");
  if (rows == 0) return 0;
  HIPO_REQUIRE(cols > 0, "rmsnorm: cols must be > 0");
  HIPO_REQUIRE(x && gamma && y && rstd, "rmsnorm: null pointer");
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  HIPO_REQUIRE(blocks <= 0x7fffffff, "rmsnorm: too many rows");
  const dim3 grid(static_cast<unsigned>(blocks));
  const int64_t nch = (cols + kChunk - 1) / kChunk;
  const bool vec = cols % 8 == 0 && nch <= 8 && aligned16(x) &&
                   aligned16(gamma) && aligned16(y);
  if (vec) {
    HIPO_NCH_SWITCH(nch, rmsnorm_rows, grid, stream, x, gamma, y, rstd, rows,
                    cols, eps);
  } else {
    rmsnorm_rows_scalar<<<grid, dim3(256), 0, stream>>>(x, gamma, y, rstd, rows,
                                                        cols, eps);
  }
  return check_launch("rmsnorm_bf16");
}
