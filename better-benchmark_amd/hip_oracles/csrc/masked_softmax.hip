// Scaled, additively masked softmax over the last dim, bf16 in / bf16 out.
//
// Semantics (eager op order of softmax(x * scale + mask, -1) on bf16):
//   s = bf16(bf16(x * scale) + mask[q, :])       (each eager bf16 op rounds)
//   out = bf16(exp(s - max(s)) / sum(exp(s - max(s))))   (fp32 max and sum)
// When `scale` is a power of two, x * scale is exact in fp32 and the first
// rounding is the identity, so it is skipped.
//
// One wave64 per row, four rows per 256-thread workgroup.  A row of K
// elements is held in registers: lane l owns elements [c*512 + 8l, +8) for
// chunk c, read and written with one 16-byte access per chunk (each access
// instruction covers 1 KiB of contiguous row).  The mask row (mask[q, :],
// q = row % Q) is re-read by every batch entry and stays cache-resident.
// Row max and row sum use DPP wave reductions.  HBM-bound: algorithmic bytes
// per element = 2 (read) + 2 (write), plus the mask once.
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kChunk = 8 * kWave;  // elements per 16-byte-per-lane chunk
constexpr float kLog2e = 1.4426950408889634f;

template <int NCH, bool ROUND_SCALE>
__global__ __launch_bounds__(256) void masked_softmax_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, int64_t rows, int64_t Q, int64_t K,
    int64_t mask_stride, float scale) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const int64_t q = row % Q;
  const uint16_t* xr = x + row * K;
  const uint16_t* mr = mask + q * mask_stride;
  uint16_t* orow = out + row * K;

  uint4 xv[NCH], mv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < K) {
      xv[c] = *reinterpret_cast<const uint4*>(xr + col);
      mv[c] = *reinterpret_cast<const uint4*>(mr + col);
    } else {
      xv[c] = make_uint4(0u, 0u, 0u, 0u);
      mv[c] = make_uint4(0u, 0u, 0u, 0u);
    }
  }

  float s[NCH][8];
  float m = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    const uint32_t xw[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    const uint32_t mw[4] = {mv[c].x, mv[c].y, mv[c].z, mv[c].w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      float a0 = bf16lo(xw[d]) * scale;
      float a1 = bf16hi(xw[d]) * scale;
      if (ROUND_SCALE) {
        const uint32_t r = pack_bf16x2(a0, a1);
        a0 = bf16lo(r);
        a1 = bf16hi(r);
      }
      const uint32_t t = pack_bf16x2(a0 + bf16lo(mw[d]), a1 + bf16hi(mw[d]));
      s[c][2 * d] = bf16lo(t);
      s[c][2 * d + 1] = bf16hi(t);
    }
    if (col >= K) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s[c][e] = -__builtin_inff();
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, s[c][e]);
  }
  m = wave_max(m);

  // exp(s - m) = 2^(s*log2e - m*log2e); (-inf) - (-inf) gives NaN exactly as
  // the eager formula does for an all-masked row.
  const float ml = m * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[c][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][e], kLog2e, -ml));
      sum += s[c][e];
    }
  }
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = static_cast<int64_t>(c) * kChunk + lane * 8;
    if (col < K) {
      uint4 o;
      o.x = pack_bf16x2(s[c][0] * inv, s[c][1] * inv);
      o.y = pack_bf16x2(s[c][2] * inv, s[c][3] * inv);
      o.z = pack_bf16x2(s[c][4] * inv, s[c][5] * inv);
      o.w = pack_bf16x2(s[c][6] * inv, s[c][7] * inv);
      *reinterpret_cast<uint4*>(orow + col) = o;
    }
  }
}

// Any K / alignment: one wave per row, three passes over the row (max, sum,
// write) with scalar accesses.
__global__ __launch_bounds__(256) void masked_softmax_rows_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, int64_t rows, int64_t Q, int64_t K,
    int64_t mask_stride, float scale, int round_scale) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t q = row % Q;
  const uint16_t* xr = x + row * K;
  const uint16_t* mr = mask + q * mask_stride;
  uint16_t* orow = out + row * K;
  auto score = [&](int64_t j) {
    float a = bf16_to_f32(xr[j]) * scale;
    if (round_scale) a = round_bf16(a);
    return round_bf16(a + bf16_to_f32(mr[j]));
  };
  float m = -__builtin_inff();
  for (int64_t j = lane; j < K; j += kWave) m = fmaxf(m, score(j));
  m = wave_max(m);
  const float ml = m * kLog2e;
  float sum = 0.f;
  for (int64_t j = lane; j < K; j += kWave)
    sum += __builtin_amdgcn_exp2f(__builtin_fmaf(score(j), kLog2e, -ml));
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  for (int64_t j = lane; j < K; j += kWave) {
    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(score(j), kLog2e, -ml));
    orow[j] = static_cast<uint16_t>(pack_bf16x2(e * inv, 0.f) & 0xffffu);
  }
}

bool is_power_of_two(float v) {
  if (!(v > 0.0f) || v == __builtin_inff()) return false;
  int e = 0;
  return __builtin_frexpf(v, &e) == 0.5f;
}

template <int NCH>
void launch_vec(bool round_scale, dim3 grid, hipStream_t stream,
                const uint16_t* x, const uint16_t* mask, uint16_t* out,
                int64_t rows, int64_t Q, int64_t K, int64_t ms, float scale) {
  if (round_scale) {
    masked_softmax_rows<NCH, true><<<grid, dim3(256), 0, stream>>>(
        x, mask, out, rows, Q, K, ms, scale);
  } else {
    masked_softmax_rows<NCH, false><<<grid, dim3(256), 0, stream>>>(
        x, mask, out, rows, Q, K, ms, scale);
  }
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_scaled_masked_softmax_bf16(const uint16_t* x,
                                               const uint16_t* mask,
                                               uint16_t* out, int64_t batch,
                                               int64_t q, int64_t k,
                                               int64_t mask_row_stride,
                                               float scale,
                                               hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(batch >= 0 && q >= 0 && k >= 0, "masked_softmax: negative size");
  if (batch == 0 || q == 0 || k == 0) return 0;
  HIPO_REQUIRE(x && mask && out, "masked_softmax: null pointer");
  HIPO_REQUIRE(mask_row_stride >= k, "masked_softmax: mask_row_stride < k");
  const int64_t rows = batch * q;
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  HIPO_REQUIRE(blocks <= 0x7fffffff, "masked_softmax: too many rows");
  const dim3 grid(static_cast<unsigned>(blocks));
  const bool round_scale = !is_power_of_two(scale);
  const int64_t nch = (k + kChunk - 1) / kChunk;
  const bool vec = (k % 8 == 0) && (mask_row_stride % 8 == 0) && nch <= 8 &&
                   (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(mask) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  if (vec) {
    switch (nch) {
      case 1: launch_vec<1>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      case 2: launch_vec<2>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      case 3: launch_vec<3>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      case 4: launch_vec<4>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      case 5: launch_vec<5>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      case 6: launch_vec<6>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      case 7: launch_vec<7>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
      default: launch_vec<8>(round_scale, grid, stream, x, mask, out, rows, q, k, mask_row_stride, scale); break;
    }
  } else {
    masked_softmax_rows_scalar<<<grid, dim3(256), 0, stream>>>(
        x, mask, out, rows, q, k, mask_row_stride, scale, round_scale ? 1 : 0);
  }
  return check_launch("scaled_masked_softmax_bf16");
}
