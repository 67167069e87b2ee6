// Row normalisations over the last dim, bf16 in / bf16 out, fp32 statistics:
//   residual-add LayerNorm  (outputs h, y, mean, rstd)
//   RMSNorm                 (outputs y, rstd)
//
// Layout (row_layout.h): W waves per row, the row held in registers between
// its statistics and its output, non-temporal 16-byte streaming accesses,
// gamma / beta re-read by every row from cache.
//
// LayerNorm statistics are over the bf16-rounded h (the eager op order).
// Each wave computes an exact two-pass (count, mean, M2) over its own
// values in registers; the W triples of a row are merged through LDS in
// closed form (the k-group form of Chan's formula: one division), in a
// fixed order (deterministic).  RMSNorm adds the
// W wave sums of squares in a fixed order.
//
// HBM-bound.  Algorithmic bytes per row (cols = C):
//   residual LayerNorm: 2C (x) + 2C (residual) + 2C (h) + 2C (y) + 8
//   RMSNorm:            2C (x) + 2C (y) + 4
#include <type_traits>

#include "row_layout.h"
#include "welford.h"

namespace hipo {
namespace {

template <int U, int WT>
__global__ __launch_bounds__(kRowMaxThreads) void residual_layernorm_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    uint16_t* __restrict__ h, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t rows,
    int64_t cols, float eps, int w_arg, int rpb_arg) {
  const int waves_per_row = WT > 0 ? WT : w_arg;
  const int rows_per_block = WT > 0 ? kRowMaxWaves / WT : rpb_arg;
  __shared__ Welford part[kRowMaxWaves];
  const RowPlace p = row_place(waves_per_row, rows_per_block, rows);
  const int64_t base = p.row * cols;

  u32x4_t hv[U], rv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t col = row_group_col(u, waves_per_row, p);
    hv[u] = row_load_stream(x + base, col, cols);
    rv[u] = row_load_stream(res + base, col, cols);
  }

  // h = bf16(x + residual); statistics use the bf16-rounded h.  Groups past
  // the row end are zero and add nothing to the sum.
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      hv[u][d] = pack_bf16x2(bf16lo(hv[u][d]) + bf16lo(rv[u][d]),
                             bf16hi(hv[u][d]) + bf16hi(rv[u][d]));
      sum += bf16lo(hv[u][d]) + bf16hi(hv[u][d]);
    }
    const int64_t col = row_group_col(u, waves_per_row, p);
    if (h != nullptr && p.valid && col < cols) row_store_stream(h + base, col, hv[u]);
  }
  const float n = static_cast<float>(row_wave_count(U, waves_per_row, p, cols));
  const float wmean = n > 0.f ? wave_sum(sum) / n : 0.f;
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool in = row_group_col(u, waves_per_row, p) < cols;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = in ? bf16lo(hv[u][d]) - wmean : 0.f;
      const float b = in ? bf16hi(hv[u][d]) - wmean : 0.f;
      sq = __builtin_fmaf(a, a, sq);
      sq = __builtin_fmaf(b, b, sq);
    }
  }
  Welford t{n, wmean, wave_sum(sq)};
  if (waves_per_row > 1) {
    // The W wave triples of the row merged in closed form, in wave order:
    // N = sum n_k, mean = sum n_k mean_k / N, M2 = sum M2_k + n_k (mean_k -
    // mean)^2 (one division; waves without values add zero).
    if (p.lane == 0) part[p.wave] = t;
    __syncthreads();
    const int first = p.wave - p.w;
    float nn = 0.f, s1 = 0.f;
    for (int k = 0; k < waves_per_row; ++k) {
      nn += part[first + k].n;
      s1 = __builtin_fmaf(part[first + k].n, part[first + k].mean, s1);
    }
    const float mu = s1 / nn;
    float m2 = 0.f;
    for (int k = 0; k < waves_per_row; ++k) {
      const float d = part[first + k].mean - mu;
      m2 += __builtin_fmaf(part[first + k].n * d, d, part[first + k].m2);
    }
    t = Welford{nn, mu, m2};
  }
  const float mean = t.mean;
  const float rstd = 1.0f / __builtin_sqrtf(t.m2 / static_cast<float>(cols) + eps);
  const float shift = -mean * rstd;

#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t col = row_group_col(u, waves_per_row, p);
    const u32x4_t gv = row_load_cached(gamma, col, cols);
    const u32x4_t bv = row_load_cached(beta, col, cols);
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float n0 = __builtin_fmaf(bf16lo(hv[u][d]), rstd, shift);
      const float n1 = __builtin_fmaf(bf16hi(hv[u][d]), rstd, shift);
      o[d] = pack_bf16x2(__builtin_fmaf(n0, bf16lo(gv[d]), bf16lo(bv[d])),
                         __builtin_fmaf(n1, bf16hi(gv[d]), bf16hi(bv[d])));
    }
    if (p.valid && col < cols) row_store_stream(y + base, col, o);
  }
  if (p.valid && p.w == 0 && p.lane == 0) {
    if (mean_out != nullptr) mean_out[p.row] = mean;
    if (rstd_out != nullptr) rstd_out[p.row] = rstd;
  }
}

// MODE 0 (torch rms_norm): y = bf16(h * rstd * gamma * scale), one rounding.
// MODE 1 (HF T5 op order): t = bf16(h * rstd); u = bf16(gamma * t);
//                          y = scale == 1 ? u : bf16(u * scale).
// With a residual, h = bf16(x + residual) (the eager bf16 add), else h = x.
template <int U, int WT, bool RES, int MODE>
__global__ __launch_bounds__(kRowMaxThreads) void rmsnorm_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ h, uint16_t* __restrict__ y,
    float* __restrict__ rstd_out, int64_t rows, int64_t cols, float eps,
    float scale, int w_arg, int rpb_arg) {
  const int waves_per_row = WT > 0 ? WT : w_arg;
  const int rows_per_block = WT > 0 ? kRowMaxWaves / WT : rpb_arg;
  __shared__ float part[kRowMaxWaves];
  const RowPlace p = row_place(waves_per_row, rows_per_block, rows);
  const int64_t base = p.row * cols;

  u32x4_t xv[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    xv[u] = row_load_stream(x + base, row_group_col(u, waves_per_row, p), cols);
  if (RES) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const u32x4_t rv =
          row_load_stream(res + base, row_group_col(u, waves_per_row, p), cols);
#pragma unroll
      for (int d = 0; d < 4; ++d)
        xv[u][d] = pack_bf16x2(bf16lo(xv[u][d]) + bf16lo(rv[d]),
                               bf16hi(xv[u][d]) + bf16hi(rv[d]));
      const int64_t col = row_group_col(u, waves_per_row, p);
      if (h != nullptr && p.valid && col < cols) row_store_stream(h + base, col, xv[u]);
    }
  }
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = bf16lo(xv[u][d]);
      const float b = bf16hi(xv[u][d]);
      sq = __builtin_fmaf(a, a, sq);
      sq = __builtin_fmaf(b, b, sq);
    }
  }
  sq = wave_sum(sq);
  if (waves_per_row > 1) {
    if (p.lane == 0) part[p.wave] = sq;
    __syncthreads();
    const int first = p.wave - p.w;
    sq = part[first];
    for (int k = 1; k < waves_per_row; ++k) sq += part[first + k];
  }
  const float rstd = 1.0f / __builtin_sqrtf(sq / static_cast<float>(cols) + eps);

  // The scale test is hoisted out of the per-element loop (one uniform
  // branch, two copies of the store loop).
  auto store = [&](auto scaled) {
    constexpr bool kScaled = decltype(scaled)::value;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t col = row_group_col(u, waves_per_row, p);
      const u32x4_t gv = row_load_cached(gamma, col, cols);
      u32x4_t o;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float a = bf16lo(xv[u][d]) * rstd, b = bf16hi(xv[u][d]) * rstd;
        if constexpr (MODE == 0) {
          a *= bf16lo(gv[d]);
          b *= bf16hi(gv[d]);
          if constexpr (kScaled) {
            a *= scale;
            b *= scale;
          }
          o[d] = pack_bf16x2(a, b);
        } else {
          const uint32_t t = pack_bf16x2(a, b);
          uint32_t w = pack_bf16x2(bf16lo(gv[d]) * bf16lo(t), bf16hi(gv[d]) * bf16hi(t));
          if constexpr (kScaled) w = pack_bf16x2(bf16lo(w) * scale, bf16hi(w) * scale);
          o[d] = w;
        }
      }
      if (p.valid && col < cols) row_store_stream(y + base, col, o);
    }
  };
  if (scale != 1.0f) {
    store(std::true_type{});
  } else {
    store(std::false_type{});
  }
  if (rstd_out != nullptr && p.valid && p.w == 0 && p.lane == 0) rstd_out[p.row] = rstd;
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
      static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float sum = 0.f;
  for (int64_t j = lane; j < cols; j += kWave) {
    const float hv = round_bf16(bf16_to_f32(x[base + j]) + bf16_to_f32(res[base + j]));
    if (h != nullptr) h[base + j] = static_cast<uint16_t>(pack_bf16x2(hv, 0.f) & 0xffffu);
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
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

__global__ __launch_bounds__(256) void rmsnorm_rows_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ h, uint16_t* __restrict__ y,
    float* __restrict__ rstd_out, int64_t rows, int64_t cols, float eps,
    float scale, int mode) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  auto hval = [&](int64_t j) {
    const float a = bf16_to_f32(x[base + j]);
    return res != nullptr ? round_bf16(a + bf16_to_f32(res[base + j])) : a;
  };
  float sq = 0.f;
  for (int64_t j = lane; j < cols; j += kWave) {
    const float a = hval(j);
    sq = __builtin_fmaf(a, a, sq);
    if (h != nullptr) h[base + j] = static_cast<uint16_t>(pack_bf16x2(a, 0.f) & 0xffffu);
  }
  const float rstd =
      1.0f / __builtin_sqrtf(wave_sum(sq) / static_cast<float>(cols) + eps);
  for (int64_t j = lane; j < cols; j += kWave) {
    float v = hval(j) * rstd;
    if (mode == 0) {
      v = v * bf16_to_f32(gamma[j]);
      if (scale != 1.0f) v *= scale;
    } else {
      v = round_bf16(bf16_to_f32(gamma[j]) * round_bf16(v));
      if (scale != 1.0f) v = v * scale;
    }
    y[base + j] = static_cast<uint16_t>(pack_bf16x2(v, 0.f) & 0xffffu);
  }
  if (rstd_out != nullptr && lane == 0) rstd_out[row] = rstd;
}

// Rows of exactly KC columns (4096, the config): NR row slots per
// workgroup, W waves per row (KC / (8 W 64) groups of 16 bytes per lane and
// stream), RPW rows per slot (rows b * NR * RPW + rr + NR * j, j < RPW),
// their loads issued together; row index from the block index without
// division.  gamma and beta: STAGE = staged once per workgroup in LDS (the
// barrier publishes them), else each lane loads its own groups from the
// cache with the row.  Same arithmetic as residual_layernorm_rows
// (per-wave two-pass statistics of the bf16 h, closed-form merge of the W
// triples in wave order).
template <int KC, int W, int NR, int RPW, bool STAGE>
__global__ __launch_bounds__(W * NR * 64) void residual_layernorm_k(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    uint16_t* __restrict__ h, uint16_t* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t rows, float eps) {
  constexpr int kThreads = W * NR * kWave;
  constexpr int G = KC / kRowGroup;
  constexpr int U = G / (W * kWave);
  static_assert(U * W * kWave == G, "row shape");
  __shared__ __align__(16) u32x4_t gs[STAGE ? G : 1];
  __shared__ __align__(16) u32x4_t bs[STAGE ? G : 1];
  __shared__ Welford part[RPW][W * NR];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int w = wave % W;
  const int rr = wave / W;

  u32x4_t hv[RPW][U], rv[RPW][U];
  int64_t r[RPW], base[RPW];
  bool valid[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    r[j] = static_cast<int64_t>(blockIdx.x) * (NR * RPW) + rr + NR * j;
    valid[j] = r[j] < rows;
    base[j] = (valid[j] ? r[j] : rows - 1) * KC;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int col = ((u * W + w) * kWave + lane) * kRowGroup;
      hv[j][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + base[j] + col));
      rv[j][u] =
          __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(res + base[j] + col));
    }
  }
  u32x4_t gl[STAGE ? 1 : U], bl[STAGE ? 1 : U];
  if constexpr (STAGE) {
    for (int i = threadIdx.x; i < G; i += kThreads) {
      gs[i] = *reinterpret_cast<const u32x4_t*>(gamma + i * kRowGroup);
      bs[i] = *reinterpret_cast<const u32x4_t*>(beta + i * kRowGroup);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = (u * W + w) * kWave + lane;
      gl[u] = *reinterpret_cast<const u32x4_t*>(gamma + g * kRowGroup);
      bl[u] = *reinterpret_cast<const u32x4_t*>(beta + g * kRowGroup);
    }
  }

#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        hv[j][u][d] = pack_bf16x2(bf16lo(hv[j][u][d]) + bf16lo(rv[j][u][d]),
                                  bf16hi(hv[j][u][d]) + bf16hi(rv[j][u][d]));
        sum += bf16lo(hv[j][u][d]) + bf16hi(hv[j][u][d]);
      }
      if (h != nullptr && valid[j])
        __builtin_nontemporal_store(
            hv[j][u],
            reinterpret_cast<u32x4_t*>(h + base[j] + ((u * W + w) * kWave + lane) * kRowGroup));
    }
    constexpr float n = U * kRowGroup * kWave;
    const float wmean = wave_sum(sum) / n;
    float sq = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float a = bf16lo(hv[j][u][d]) - wmean;
        const float b = bf16hi(hv[j][u][d]) - wmean;
        sq = __builtin_fmaf(a, a, sq);
        sq = __builtin_fmaf(b, b, sq);
      }
    }
    const Welford t{n, wmean, wave_sum(sq)};
    if (lane == 0) part[j][wave] = t;
    __syncthreads();  // also publishes gs / bs
    const int first = rr * W;
    float nn = 0.f, s1 = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      nn += part[j][first + k].n;
      s1 = __builtin_fmaf(part[j][first + k].n, part[j][first + k].mean, s1);
    }
    const float mean = s1 / nn;
    float m2 = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const float d = part[j][first + k].mean - mean;
      m2 += __builtin_fmaf(part[j][first + k].n * d, d, part[j][first + k].m2);
    }
    const float rstd = 1.0f / __builtin_sqrtf(m2 / static_cast<float>(KC) + eps);
    const float shift = -mean * rstd;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = (u * W + w) * kWave + lane;
      const u32x4_t gv = STAGE ? gs[g] : gl[STAGE ? 0 : u];
      const u32x4_t bv = STAGE ? bs[g] : bl[STAGE ? 0 : u];
      u32x4_t o;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float n0 = __builtin_fmaf(bf16lo(hv[j][u][d]), rstd, shift);
        const float n1 = __builtin_fmaf(bf16hi(hv[j][u][d]), rstd, shift);
        o[d] = pack_bf16x2(__builtin_fmaf(n0, bf16lo(gv[d]), bf16lo(bv[d])),
                           __builtin_fmaf(n1, bf16hi(gv[d]), bf16hi(bv[d])));
      }
      if (valid[j])
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(y + base[j] + g * kRowGroup));
    }
    if (valid[j] && w == 0 && lane == 0) {
      if (mean_out != nullptr) mean_out[r[j]] = mean;
      if (rstd_out != nullptr) rstd_out[r[j]] = rstd;
    }
  }
}

// Rows of at most 1536 values held by L consecutive lanes (L a power of
// two, 8..64): a wave covers 64 / L rows, a 256-thread workgroup 256 / L
// consecutive rows.  Lane l of a row owns the 16-byte groups g = u * L + l
// (u < U), so each load instruction of a wave reads L * 16 contiguous bytes
// of every one of its rows.  Groups past the row end re-read the row's last
// group and count for nothing.  Statistics: the exact two-pass over the
// row's bf16 h (sum -> mean, then the sum of squared deviations from it),
// each reduced over the row's L lanes by seg_sum in a fixed order.  gamma
// and beta of a lane's groups are the same for every row, loaded once.
// Plans (seg_plan): rows of up to 512 values take one group per lane (L =
// the row's groups rounded up to a power of two, at least 8), rows of
// 520..1536 values 64 lanes with 2 or 3 groups when there are at least 16384
// of them; the rest take the row kernel.  Measured on MI355X (oracle runner,
// graph replays after a cache flush; the row kernel's time first):
// [131072, 144] 58.4 -> 36.9 us (8 lanes x 3 groups: 53.8), [25216, 192]
// 21.4 -> 18.4, [32768, 256] 23.6 -> 20.0, [16384, 768] 24.6 -> 23.8,
// [32768, 768] 35.8 -> 34.9, [16384, 1024] 28.4 -> 27.6; but [8192, 1024]
// 19.2 -> 20.0 and [8192, 768] 17.6 -> 18.0 (also with 8-row workgroups or
// DPP-and-readlane sums: 19.7, 19.9), and at 2048 values one wave per row
// with 4 groups lost to the row kernel's two waves with 2 (20.4 against
// 19.2 us).
template <int L, int U>
__global__ __launch_bounds__(256) void residual_layernorm_seg(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, const uint16_t* __restrict__ beta,
    uint16_t* __restrict__ h, uint16_t* __restrict__ y, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int64_t rows, int cols, float eps) {
  constexpr int kRowsPerBlock = 256 / L;
  const int l = static_cast<int>(threadIdx.x) & (L - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / L;
  const bool valid = row < rows;
  const int64_t base = (valid ? row : rows - 1) * cols;
  const int groups = cols / kRowGroup;

  u32x4_t hv[U], rv[U], gv[U], bv[U];
  bool in[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int g = u * L + l;
    in[u] = g < groups;
    const int col = (in[u] ? g : groups - 1) * kRowGroup;
    hv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + base + col));
    rv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(res + base + col));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int col = (in[u] ? u * L + l : groups - 1) * kRowGroup;
    gv[u] = *reinterpret_cast<const u32x4_t*>(gamma + col);
    bv[u] = *reinterpret_cast<const u32x4_t*>(beta + col);
  }

  // h = bf16(x + residual); the statistics use the bf16-rounded h.
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      hv[u][d] = pack_bf16x2(bf16lo(hv[u][d]) + bf16lo(rv[u][d]),
                             bf16hi(hv[u][d]) + bf16hi(rv[u][d]));
      if (in[u]) sum += bf16lo(hv[u][d]) + bf16hi(hv[u][d]);
    }
    if (h != nullptr && valid && in[u])
      row_store_stream(h + base, static_cast<int64_t>(u * L + l) * kRowGroup, hv[u]);
  }
  const float inv_n = 1.0f / static_cast<float>(cols);
  const float mean = seg_sum<L>(sum) * inv_n;
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float a = bf16lo(hv[u][d]) - mean;
      const float b = bf16hi(hv[u][d]) - mean;
      if (in[u]) sq = __builtin_fmaf(a, a, __builtin_fmaf(b, b, sq));
    }
  }
  const float rstd = 1.0f / __builtin_sqrtf(seg_sum<L>(sq) * inv_n + eps);
  const float shift = -mean * rstd;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float n0 = __builtin_fmaf(bf16lo(hv[u][d]), rstd, shift);
      const float n1 = __builtin_fmaf(bf16hi(hv[u][d]), rstd, shift);
      o[d] = pack_bf16x2(__builtin_fmaf(n0, bf16lo(gv[u][d]), bf16lo(bv[u][d])),
                         __builtin_fmaf(n1, bf16hi(gv[u][d]), bf16hi(bv[u][d])));
    }
    if (valid && in[u]) row_store_stream(y + base, static_cast<int64_t>(u * L + l) * kRowGroup, o);
  }
  if (valid && l == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

struct SegPlan {
  int lanes = 0, groups = 0;  // 0: not this kernel
};

SegPlan seg_plan(int64_t rows, int64_t cols) {
  SegPlan p;
  if (cols % kRowGroup != 0 || cols <= 0 || cols > 1536) return p;
  const int g = static_cast<int>(cols / kRowGroup);
  if (g > kWave && rows < 16384) return p;  // the row kernel's 8-row workgroups win there
  if (g <= kWave) {
    p.lanes = 8;
    while (p.lanes < g) p.lanes *= 2;
    p.groups = 1;
  } else {
    p.lanes = kWave;
    p.groups = (g + kWave - 1) / kWave;
  }
  return p;
}

template <int L, int U>
void launch_seg(int64_t rows, hipStream_t stream, const uint16_t* x, const uint16_t* residual,
                const uint16_t* gamma, const uint16_t* beta, uint16_t* h, uint16_t* y,
                float* mean, float* rstd, int cols, float eps) {
  constexpr int kRowsPerBlock = 256 / L;
  residual_layernorm_seg<L, U>
      <<<dim3(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock)), dim3(256), 0,
         stream>>>(x, residual, gamma, beta, h, y, mean, rstd, rows, cols, eps);
}

// Dispatch over the (L, U) pairs seg_plan returns.
void launch_seg_plan(const SegPlan& sp, int64_t rows, hipStream_t stream, const uint16_t* x,
                     const uint16_t* residual, const uint16_t* gamma, const uint16_t* beta,
                     uint16_t* h, uint16_t* y, float* mean, float* rstd, int cols, float eps) {
#define HIPO_SEG(L_, U_) \
  launch_seg<L_, U_>(rows, stream, x, residual, gamma, beta, h, y, mean, rstd, cols, eps)
  if (sp.groups == 1) {
    switch (sp.lanes) {
      case 8: HIPO_SEG(8, 1); break;
      case 16: HIPO_SEG(16, 1); break;
      case 32: HIPO_SEG(32, 1); break;
      default: HIPO_SEG(64, 1); break;
    }
  } else if (sp.groups == 2) {
    HIPO_SEG(64, 2);
  } else {
    HIPO_SEG(64, 3);
  }
#undef HIPO_SEG
}

// Shape of residual_layernorm_k at 4096 columns: waves per row, row slots
// per workgroup, rows per slot, gamma / beta staged in LDS.  Rows per slot,
// measured at [16384, 4096], one process: 1 row 90.2-90.8 us, 2 rows 93.4
// us, 4 rows 100.6-102.8 us.  Waves per row x slots, back to back (flat
// copy 83.1-83.4 us): 2 x 2 89.4-90.1 us, 2 x 4 89.4-89.5, 4 x 1 90.8-90.9,
// 1 x 2 94.5, 1 x 4 94.0 (94.5 with gamma / beta from the cache).
constexpr int kLnWaves = 2;
constexpr int kLnSlots = 2;
constexpr int kLayerNormRowsPerWave = 1;
constexpr bool kLnStage = true;

}  // namespace
}  // namespace hipo


extern "C" int hipo_residual_layernorm_bf16(
    const uint16_t* x, const uint16_t* residual, const uint16_t* gamma,
    const uint16_t* beta, uint16_t* h, uint16_t* y, float* mean, float* rstd,
    int64_t rows, int64_t cols, float eps, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "residual_layernorm: negative size");
  if (rows == 0) return 0;
  HIPO_REQUIRE(cols > 0, "residual_layernorm: cols must be > 0");
  HIPO_REQUIRE(x && residual && gamma && beta && y,
               "residual_layernorm: null pointer");
  RowPlan plan;
  const bool vec = cols % 8 == 0 && row_plan(cols, plan) && aligned16(x) &&
                   aligned16(residual) && aligned16(gamma) && aligned16(beta) &&
                   (h == nullptr || aligned16(h)) && aligned16(y);
  constexpr int kRowsPerBlock = kLnSlots * kLayerNormRowsPerWave;
  if (vec && cols == 4096 && (rows + kRowsPerBlock - 1) / kRowsPerBlock <= 0x7fffffff) {
    residual_layernorm_k<4096, kLnWaves, kLnSlots, kLayerNormRowsPerWave, kLnStage>
        <<<dim3(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
           dim3(kLnWaves * kLnSlots * kWave), 0, stream>>>(x, residual, gamma, beta, h, y, mean,
                                                           rstd, rows, eps);
  } else if (const SegPlan sp = vec ? seg_plan(rows, cols) : SegPlan{};
             sp.lanes > 0 && (rows + 256 / sp.lanes - 1) / (256 / sp.lanes) <= 0x7fffffff) {
    launch_seg_plan(sp, rows, stream, x, residual, gamma, beta, h, y, mean, rstd,
                    static_cast<int>(cols), eps);
  } else if (vec) {
    const int64_t blocks = (rows + plan.rows_per_block - 1) / plan.rows_per_block;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "residual_layernorm: too many rows");
    const dim3 grid(static_cast<unsigned>(blocks));
    const dim3 block(plan.threads());
#define HIPO_LN(U_, W_)                                                              \
  residual_layernorm_rows<U_, W_><<<grid, block, 0, stream>>>(                       \
      x, residual, gamma, beta, h, y, mean, rstd, rows, cols, eps, plan.waves_per_row, \
      plan.rows_per_block)
    HIPO_ROW_DISPATCH(plan, HIPO_LN);
#undef HIPO_LN
  } else {
    const int64_t blocks = (rows + 3) / 4;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "residual_layernorm: too many rows");
    residual_layernorm_rows_scalar<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
        x, residual, gamma, beta, h, y, mean, rstd, rows, cols, eps);
  }
  return check_launch("residual_layernorm_bf16");
}

namespace hipo {
namespace {

template <bool RES, int MODE>
void launch_rmsnorm(const RowPlan& plan, dim3 grid, hipStream_t stream,
                    const uint16_t* x, const uint16_t* residual,
                    const uint16_t* gamma, uint16_t* h, uint16_t* y, float* rstd,
                    int64_t rows, int64_t cols, float eps, float scale) {
  const dim3 block(plan.threads());
  const int w = plan.waves_per_row, r = plan.rows_per_block;
#define HIPO_RMS(U_, W_)                                            \
  rmsnorm_rows<U_, W_, RES, MODE><<<grid, block, 0, stream>>>(      \
      x, residual, gamma, h, y, rstd, rows, cols, eps, scale, w, r)
  HIPO_ROW_DISPATCH(plan, HIPO_RMS);
#undef HIPO_RMS
}

int rmsnorm_impl(const uint16_t* x, const uint16_t* residual, const uint16_t* gamma,
                 uint16_t* h, uint16_t* y, float* rstd, int64_t rows, int64_t cols,
                 float eps, float scale, int mode, bool require_rstd, hipStream_t stream,
                 const char* what) {
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "%s: negative size", what);
  if (rows == 0) return 0;
  HIPO_REQUIRE(cols > 0, "%s: cols must be > 0", what);
  HIPO_REQUIRE(x && gamma && y && (rstd || !require_rstd), "%s: null pointer", what);
  HIPO_REQUIRE(h == nullptr || residual != nullptr, "%s: h needs a residual", what);
  HIPO_REQUIRE(mode == 0 || mode == 1, "%s: mode must be 0 or 1", what);
  RowPlan plan;
  const bool vec = cols % 8 == 0 && row_plan(cols, plan) && aligned16(x) &&
                   aligned16(gamma) && aligned16(y) &&
                   (residual == nullptr || aligned16(residual)) && (h == nullptr || aligned16(h));
  if (vec) {
    const int64_t blocks = (rows + plan.rows_per_block - 1) / plan.rows_per_block;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "%s: too many rows", what);
    const dim3 grid(static_cast<unsigned>(blocks));
    if (residual != nullptr) {
      if (mode == 0) launch_rmsnorm<true, 0>(plan, grid, stream, x, residual, gamma, h, y, rstd, rows, cols, eps, scale);
      else launch_rmsnorm<true, 1>(plan, grid, stream, x, residual, gamma, h, y, rstd, rows, cols, eps, scale);
    } else {
      if (mode == 0) launch_rmsnorm<false, 0>(plan, grid, stream, x, residual, gamma, nullptr, y, rstd, rows, cols, eps, scale);
      else launch_rmsnorm<false, 1>(plan, grid, stream, x, residual, gamma, nullptr, y, rstd, rows, cols, eps, scale);
    }
  } else {
    const int64_t blocks = (rows + 3) / 4;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "%s: too many rows", what);
    rmsnorm_rows_scalar<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
        x, residual, gamma, h, y, rstd, rows, cols, eps, scale, mode);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma,
                                 uint16_t* y, float* rstd, int64_t rows,
                                 int64_t cols, float eps, hipStream_t stream) {
  return hipo::rmsnorm_impl(x, nullptr, gamma, nullptr, y, rstd, rows, cols, eps, 1.0f, 0,
                            true, stream, "rmsnorm_bf16");
}

extern "C" int hipo_rmsnorm_ex_bf16(const uint16_t* x, const uint16_t* residual,
                                    const uint16_t* gamma, uint16_t* h, uint16_t* y,
                                    float* rstd, int64_t rows, int64_t cols,
                                    float eps, float scale, int mode,
                                    hipStream_t stream) {
  return hipo::rmsnorm_impl(x, residual, gamma, h, y, rstd, rows, cols, eps, scale, mode,
                            false, stream, "rmsnorm_ex_bf16");
}
