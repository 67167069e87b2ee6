// Scaled, additively masked softmax over the last dim, bf16 in / bf16 out.
//
// Semantics (softmax(x * scale + mask, -1) on bf16, scores formed in fp32
// as the reference's Triton oracles and Inductor form them):
//   s = fma(x, scale, mask[q, :])                  (fp32, one rounding)
//   out = bf16(exp(s - max(s)) / sum(exp(s - max(s))))   (fp32 max and sum)
// exp is natural exp of the fp32 difference s - max(s) (as aten.exp and
// Inductor's libdevice.exp), evaluated to about one ulp by exp_f32, the
// device library's extended-precision reduction (no exp2 rewrite).  Eager
// rounds x * scale and the sum to bf16 first; with a power-of-two scale and
// a 0 / -inf mask (the causal softmax) both roundings are exact, so the
// scores are eager's; with a general bias (TrOCR) the fp32 scores are the
// reference oracle's (its oracle.py builds them from fp32 x + bias) and
// several times closer to fp64 than eager's rounded ones.
//
// Layout: rows held in registers, non-temporal 16-byte streaming accesses
// for x and out; the mask row (mask[q, :], q = row % Q) is re-read by every
// batch entry and stays cache-resident.  Row max and row sum: DPP within a
// wave, then a fixed-order combine of the wave results through LDS.  Three
// kernels by row length:
//   K <= 512: L lanes per row, 64 / L rows per access instruction, 2 KiB of
//     x per wave, reductions within lane segments, no LDS;
//   K = 1024 or 2048 (config [384, 1024, 1024]): 1 KiB of x per wave and
//     row, each wave taking RPW = 4 rows with their loads issued together,
//     the rows of one q for 4 RPW / W batch entries in a 256-thread
//     workgroup, their shared mask row loaded once and staged through LDS;
//   otherwise (or a per-batch mask the grouping cannot share): the
//     row_layout.h plan, W waves per row, 2 KiB per wave.
// HBM-bound: algorithmic bytes per element = 2 (read) + 2 (write), plus the
// mask once.
#include "row_layout.h"

namespace hipo {
namespace {

// exp(s - m): masked entries (s = -inf) give exactly 0; (-inf) - (-inf)
// gives NaN for an all-masked row, exactly as the eager formula.
__device__ __forceinline__ float exp_shifted(float s, float m) {
  // s - m <= 0 (m is the row max) or NaN, so only exp_f32's lower bound
  // needs the clamp (IEEE maximum: NaN stays NaN).
  return exp_f32(__builtin_elementwise_maximum(s - m, -104.0f));
}

template <int U, int WT>
__global__ __launch_bounds__(kRowMaxThreads) void masked_softmax_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, int64_t rows, int64_t Q, int64_t K,
    int64_t mask_stride, int64_t mask_batch_stride, int64_t heads, float scale,
    int w_arg, int rpb_arg) {
  const int waves_per_row = WT > 0 ? WT : w_arg;
  const int rows_per_block = WT > 0 ? kRowMaxWaves / WT : rpb_arg;
  __shared__ float pmax[kRowMaxWaves], psum[kRowMaxWaves];
  const RowPlace p = row_place(waves_per_row, rows_per_block, rows);
  const int64_t b = p.row / Q;
  const int64_t q = p.row - b * Q;
  const uint16_t* xr = x + p.row * K;
  const uint16_t* mr = mask + (b / heads) * mask_batch_stride + q * mask_stride;
  uint16_t* orow = out + p.row * K;

  u32x4_t xv[U], mv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t col = row_group_col(u, waves_per_row, p);
    xv[u] = row_load_stream(xr, col, K);
    mv[u] = row_load_cached(mr, col, K);
  }

  float s[U][8];
  float m = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool in = row_group_col(u, waves_per_row, p) < K;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      s[u][2 * d] = in ? __builtin_fmaf(bf16lo(xv[u][d]), scale, bf16lo(mv[u][d]))
                       : -__builtin_inff();
      s[u][2 * d + 1] = in ? __builtin_fmaf(bf16hi(xv[u][d]), scale, bf16hi(mv[u][d]))
                           : -__builtin_inff();
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, s[u][e]);
  }
  m = wave_max(m);
  if (waves_per_row > 1) {
    if (p.lane == 0) pmax[p.wave] = m;
    __syncthreads();
    const int first = p.wave - p.w;
    m = pmax[first];
    for (int k = 1; k < waves_per_row; ++k) m = fmaxf(m, pmax[first + k]);
  }

  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[u][e] = exp_shifted(s[u][e], m);
      sum += s[u][e];
    }
  }
  sum = wave_sum(sum);
  if (waves_per_row > 1) {
    if (p.lane == 0) psum[p.wave] = sum;
    __syncthreads();
    const int first = p.wave - p.w;
    sum = psum[first];
    for (int k = 1; k < waves_per_row; ++k) sum += psum[first + k];
  }
  const float inv = 1.0f / sum;

#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t col = row_group_col(u, waves_per_row, p);
    u32x4_t o;
    o[0] = pack_bf16x2(s[u][0] * inv, s[u][1] * inv);
    o[1] = pack_bf16x2(s[u][2] * inv, s[u][3] * inv);
    o[2] = pack_bf16x2(s[u][4] * inv, s[u][5] * inv);
    o[3] = pack_bf16x2(s[u][6] * inv, s[u][7] * inv);
    if (p.valid && col < K) row_store_stream(orow, col, o);
  }
}

// Short rows (K <= 512): a row owns L = 2^j lanes, one 16-byte group each,
// so one access instruction of a wave covers 64 / L rows (1 KiB when
// K = 8 L).  Lane l holds group l % L of rows (wave * V + v) * (64 / L) +
// l / L, v = 0 .. V-1: V = 2 rows per lane keep 2 KiB of x per wave in
// flight.  Rows past the last re-read the last row and store nothing; lanes
// past K load the row's last group and score -inf.  32-bit row arithmetic
// (the host checks rows < 2^31); row / Q and batch / heads by multiply-high
// constants (TrOCR [1024, 256, 256]: 44.5 against 44.8-45.1 us with the
// division sequences, median 44.8-46.1 against 47.3-47.9; K = 512 -0.4 %,
// K = 128 +1.5 %).
// Measured on MI355X (steady state, % of 8 TB/s): K = 256 with 16-head
// bias groups 77.9 % (the long-row layout: 34 %), K = 512 79.6 %, K = 128
// and 64 about 80 %; V = 1 or 4 and 512-thread workgroups were 1-7 points
// lower.  For K = 1024 this layout (one wave per row, 2 groups per lane)
// measured the same as the row-plan kernel (75.7-76.2 % against 76.6 %), so
// longer rows use the kernels below.
constexpr int kShortV = 2;
constexpr int kShortThreads = 256;

template <int L>
__global__ __launch_bounds__(kShortThreads) void masked_softmax_short_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, uint32_t rows, uint32_t Q, DivMagic q_div, int K,
    int64_t mask_stride, int64_t mask_batch_stride, DivMagic heads_div, float scale) {
  constexpr int RI = kWave / L;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t wave = blockIdx.x * (kShortThreads / kWave) + (threadIdx.x >> 6);
  const int col = (lane % L) * kRowGroup;
  const bool col_in = col < K;
  const int c = col_in ? col : K - kRowGroup;

  uint32_t row[kShortV];
  u32x4_t xv[kShortV], mv[kShortV];
#pragma unroll
  for (int v = 0; v < kShortV; ++v) {
    row[v] = (wave * kShortV + v) * RI + lane / L;
    const uint32_t r = row[v] < rows ? row[v] : rows - 1;
    const uint32_t b = div_by(r, q_div);
    const uint32_t q = r - b * Q;
    const uint16_t* mr = mask + static_cast<int64_t>(div_by(b, heads_div)) * mask_batch_stride +
                         static_cast<int64_t>(q) * mask_stride;
    xv[v] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(x + static_cast<int64_t>(r) * K + c));
    mv[v] = *reinterpret_cast<const u32x4_t*>(mr + c);
  }

#pragma unroll
  for (int v = 0; v < kShortV; ++v) {
    float s[8];
    float m = -__builtin_inff();
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      s[2 * d] = col_in ? __builtin_fmaf(bf16lo(xv[v][d]), scale, bf16lo(mv[v][d]))
                        : -__builtin_inff();
      s[2 * d + 1] = col_in ? __builtin_fmaf(bf16hi(xv[v][d]), scale, bf16hi(mv[v][d]))
                            : -__builtin_inff();
      m = fmaxf(m, fmaxf(s[2 * d], s[2 * d + 1]));
    }
    m = seg_max<L>(m);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[e] = exp_shifted(s[e], m);
      sum += s[e];
    }
    const float inv = 1.0f / seg_sum<L>(sum);
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = pack_bf16x2(s[2 * d] * inv, s[2 * d + 1] * inv);
    if (row[v] < rows && col_in)
      __builtin_nontemporal_store(
          o, reinterpret_cast<u32x4_t*>(out + static_cast<int64_t>(row[v]) * K + col));
  }
}

template <int L>
void launch_short(dim3 grid, hipStream_t stream, const uint16_t* x, const uint16_t* mask,
                  uint16_t* out, int64_t rows, int64_t Q, int64_t K, int64_t ms, int64_t mbs,
                  int64_t heads, float scale) {
  const auto r = static_cast<uint32_t>(rows);
  const auto q = static_cast<uint32_t>(Q);
  const DivMagic qd = div_magic(q), hd = div_magic(static_cast<uint32_t>(heads));
  masked_softmax_short_rows<L><<<grid, dim3(kShortThreads), 0, stream>>>(
      x, mask, out, r, q, qd, static_cast<int>(K), ms, mbs, hd, scale);
}

// Rows of exactly K = 1024 or 2048 (KC, a compile-time constant):
// 256-thread workgroups, W = KC / 512 waves per row (one 16-byte group per
// lane: 1 KiB of x per wave and row, no idle lanes), NR = 4 / W row slots
// per workgroup, RPW rows per slot.  Workgroup (q, y, z) of the 3-D grid
// takes the rows (b0 + i) * Q + q, i < NR * RPW, b0 = (z * gy + y) * NR *
// RPW: the same q of NR * RPW consecutive batch entries, which share one
// mask row; slot rr holds entries b0 + rr + NR * j, j < RPW, whose loads a
// wave issues together before working through them.  z is the mask's batch
// group (offset z * mask_batch_stride; a single z when the mask is
// broadcast over batch) and gy its workgroups along y, so the kernel does
// no integer division; x is fastest, so dispatch order walks q in memory
// order.  The mask row (2 KC bytes, 2 KC / 256 per thread) is loaded once
// per workgroup, issued before the x loads, and staged through LDS; row max
// and sum combine the W wave results through LDS in a fixed order.  Rows
// past the batch end (NR * RPW not dividing a broadcast batch) re-read the
// last batch entry and store nothing.
// With the accurate exp (exp_f32: about 9 issue slots per element against
// 5 for a bare exp2) one row per wave ran at 288-291 us at [384, 1024,
// 1024]; issuing 2 / 4 / 8 / 16 rows' loads per wave 280 / 271-276 /
// 275-280 / 303-306 us (the bare exp2 form, one row per wave, 269-273 us on
// the same boxes).
// Measured on MI355X (graph loop, rotating buffers, 2 B read + 2 B written
// per element, % of 8 TB/s), [384, 1024, 1024]: one wave per row with every
// wave reading its own mask row (the row-plan kernel) 261.6-263.5 us
// (76.6-77.0 %); this layout with the block index split by division 272.2
// us, with a 3-D grid and a runtime K 252.7-255.0 us, with K fixed 245.4
// us = a flat copy of the same bytes; 512-thread workgroups (NR = 4 or 8)
// 260-267 us.  [192, 1024, 2048]: 258.7-260.1 us against 253.3 us.  With a
// runtime K and idle lanes (K = 776, 1032) the layout lost 8-15 % to the
// row-plan kernel, so other row lengths stay there.
template <int KC, int RPW>
__global__ __launch_bounds__(256) void masked_softmax_shared_mask(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, uint32_t batch, uint32_t Q, uint32_t gy,
    int64_t mask_stride, int64_t mask_batch_stride, float scale) {
  constexpr int W = KC / 512;
  constexpr int NR = 4 / W;
  static_assert(W * NR * kWave == 256 && W * kWave * kRowGroup == KC, "full rows");
  constexpr int kStageWords = KC / 512;  // 32-bit words of the mask row per thread
  __shared__ __align__(16) uint32_t mrow[KC / 2];  // read back as 16-byte groups
  __shared__ float pmax[RPW][W * NR], psum[RPW][W * NR];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int w = wave % W;
  const int rr = wave / W;
  const uint32_t q = blockIdx.x;
  // The workgroup's NR * RPW rows: batch entries b0 + rr + NR * i of query q;
  // wave (rr, w) takes the RPW rows of slot rr, all loads issued up front.
  const uint32_t b0 = (blockIdx.z * gy + blockIdx.y) * (NR * RPW) + rr;

  const uint16_t* mr = mask + blockIdx.z * mask_batch_stride +
                       static_cast<int64_t>(q) * mask_stride;
  const int st = static_cast<int>(threadIdx.x) * kStageWords;  // first word staged
  uint32_t mval[kStageWords];
  if constexpr (kStageWords == 2) {
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(mr + 2 * st);
    mval[0] = v[0];
    mval[1] = v[1];
  } else {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(mr + 2 * st);
#pragma unroll
    for (int i = 0; i < 4; ++i) mval[i] = v[i];
  }
  const int col = (w * kWave + lane) * kRowGroup;
  u32x4_t xv[RPW];
  int64_t row[RPW];
  bool row_ok[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const uint32_t b = b0 + NR * i;
    row_ok[i] = b < batch;
    // Rows past the batch end re-read the last batch entry and store nothing.
    row[i] = static_cast<int64_t>(row_ok[i] ? b : batch - 1) * Q + q;
    xv[i] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(x + row[i] * KC + col));
  }
#pragma unroll
  for (int i = 0; i < kStageWords; ++i) mrow[st + i] = mval[i];
  __syncthreads();
  const u32x4_t mv = *reinterpret_cast<const u32x4_t*>(&mrow[col / 2]);

#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    float s[8];
    float lmax = -__builtin_inff();  // NaN-propagating: NaN if any score is
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      s[2 * d] = __builtin_fmaf(bf16lo(xv[i][d]), scale, bf16lo(mv[d]));
      s[2 * d + 1] = __builtin_fmaf(bf16hi(xv[i][d]), scale, bf16hi(mv[d]));
      lmax = __builtin_elementwise_maximum(
          lmax, __builtin_elementwise_maximum(s[2 * d], s[2 * d + 1]));
    }
    float m = wave_max(lmax);  // fmaxf: the row max of the non-NaN scores
    if (lane == 0) pmax[i][wave] = m;
    __syncthreads();
    m = pmax[i][rr * W];
#pragma unroll
    for (int k = 1; k < W; ++k) m = fmaxf(m, pmax[i][rr * W + k]);

    // A lane whose 8 scores are all -inf (a fully masked group: the causal
    // mask's upper triangle makes whole waves of them) has exp = 0 for each;
    // a NaN score makes lmax NaN, so it still goes through exp and poisons
    // the row as in eager.
    float sum = 0.f;
    if (lmax == -__builtin_inff()) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = 0.f;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[e] = exp_shifted(s[e], m);
        sum += s[e];
      }
    }
    sum = wave_sum(sum);
    if (lane == 0) psum[i][wave] = sum;
    __syncthreads();
    sum = psum[i][rr * W];
#pragma unroll
    for (int k = 1; k < W; ++k) sum += psum[i][rr * W + k];
    const float inv = 1.0f / sum;

    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = pack_bf16x2(s[2 * d] * inv, s[2 * d + 1] * inv);
    if (row_ok[i])
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(out + row[i] * KC + col));
  }
}

// Rows per wave of the shared-mask kernel (consecutive rows of one query in
// steps of NR batch entries; their loads are issued together).
constexpr int kSharedMaskRowsPerWave = 4;

// Launch shape of the shared-mask kernel: its row length (1024 or 2048; 0
// when the kernel does not apply) and the 3-D grid.  It does not apply to
// other K, to a per-batch mask whose heads groups the NR * RPW rows of a workgroup do not
// divide, or to grids beyond the y / z limits.
struct SharedMaskPlan {
  int k = 0;
  uint32_t gy = 0;  // workgroups along y per mask batch group
  dim3 grid;
};

SharedMaskPlan shared_mask_plan(int64_t batch, int64_t Q, int64_t K, int64_t mbs,
                                int64_t heads) {
  SharedMaskPlan plan;
  if ((K != 1024 && K != 2048) || Q > 0x7fffffff) return plan;
  const int nr = (K == 1024 ? 2 : 1) * kSharedMaskRowsPerWave;  // rows per workgroup
  int64_t gy, gz;
  if (mbs == 0) {
    gy = (batch + nr - 1) / nr;
    gz = 1;
  } else {
    if (heads % nr != 0) return plan;
    gy = heads / nr;
    gz = batch / heads;
  }
  if (gy > 65535 || gz > 65535) return plan;
  plan.k = static_cast<int>(K);
  plan.gy = static_cast<uint32_t>(gy);
  plan.grid = dim3(static_cast<unsigned>(Q), static_cast<unsigned>(gy),
                   static_cast<unsigned>(gz));
  return plan;
}

template <int KC>
void launch_shared_mask(const SharedMaskPlan& plan, hipStream_t stream, const uint16_t* x,
                        const uint16_t* mask, uint16_t* out, int64_t batch, int64_t Q,
                        int64_t ms, int64_t mbs, float scale) {
  masked_softmax_shared_mask<KC, kSharedMaskRowsPerWave><<<plan.grid, dim3(256), 0, stream>>>(
      x, mask, out, static_cast<uint32_t>(batch), static_cast<uint32_t>(Q), plan.gy, ms, mbs,
      scale);
}

// Any K / alignment: one wave per row, three passes over the row (max, sum,
// write) with scalar accesses.
__global__ __launch_bounds__(256) void masked_softmax_rows_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, int64_t rows, int64_t Q, int64_t K,
    int64_t mask_stride, int64_t mask_batch_stride, int64_t heads, float scale) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =
      static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = row / Q;
  const int64_t q = row - b * Q;
  const uint16_t* xr = x + row * K;
  const uint16_t* mr = mask + (b / heads) * mask_batch_stride + q * mask_stride;
  uint16_t* orow = out + row * K;
  auto score = [&](int64_t j) {
    return __builtin_fmaf(bf16_to_f32(xr[j]), scale, bf16_to_f32(mr[j]));
  };
  float m = -__builtin_inff();
  for (int64_t j = lane; j < K; j += kWave) m = fmaxf(m, score(j));
  m = wave_max(m);
  float sum = 0.f;
  for (int64_t j = lane; j < K; j += kWave)
    sum += exp_shifted(score(j), m);
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  for (int64_t j = lane; j < K; j += kWave) {
    const float e = exp_shifted(score(j), m);
    orow[j] = static_cast<uint16_t>(pack_bf16x2(e * inv, 0.f) & 0xffffu);
  }
}

template <int U, int WT>
void launch_vec(dim3 grid, const RowPlan& plan, hipStream_t stream, const uint16_t* x,
                const uint16_t* mask, uint16_t* out, int64_t rows, int64_t Q, int64_t K,
                int64_t ms, int64_t mbs, int64_t heads, float scale) {
  masked_softmax_rows<U, WT><<<grid, dim3(plan.threads()), 0, stream>>>(
      x, mask, out, rows, Q, K, ms, mbs, heads, scale, plan.waves_per_row, plan.rows_per_block);
}

}  // namespace
}  // namespace hipo

namespace hipo {
namespace {

int softmax_impl(const uint16_t* x, const uint16_t* mask, uint16_t* out, int64_t batch,
                 int64_t q, int64_t k, int64_t mask_row_stride, int64_t mask_batch_stride,
                 int64_t heads, float scale, hipStream_t stream, const char* what) {
  clear_error();
  HIPO_REQUIRE(batch >= 0 && q >= 0 && k >= 0, "%s: negative size", what);
  if (batch == 0 || q == 0 || k == 0) return 0;
  HIPO_REQUIRE(x && mask && out, "%s: null pointer", what);
  HIPO_REQUIRE(mask_row_stride >= k, "%s: mask_row_stride < k", what);
  HIPO_REQUIRE(heads >= 1 && batch % heads == 0, "%s: heads must divide batch", what);
  HIPO_REQUIRE(mask_batch_stride >= 0, "%s: negative mask_batch_stride", what);
  const int64_t rows = batch * q;
  RowPlan plan;
  const bool vec = (k % 8 == 0) && (mask_row_stride % 8 == 0) &&
                   (mask_batch_stride % 8 == 0) && row_plan(k, plan) && aligned16(x) &&
                   aligned16(mask) && aligned16(out);
  const int lanes = short_row_lanes(k);
  if (vec && lanes > 0 && rows < (int64_t{1} << 31)) {
    const int64_t rows_per_block = int64_t{kShortV} * (kWave / lanes) * (kShortThreads / kWave);
    const dim3 grid(static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block));
#define HIPO_SHORT(L_)                                                                  \
  launch_short<L_>(grid, stream, x, mask, out, rows, q, k, mask_row_stride, mask_batch_stride, \
                   heads, scale)
    switch (lanes) {
      case 1: HIPO_SHORT(1); break;
      case 2: HIPO_SHORT(2); break;
      case 4: HIPO_SHORT(4); break;
      case 8: HIPO_SHORT(8); break;
      case 16: HIPO_SHORT(16); break;
      case 32: HIPO_SHORT(32); break;
      default: HIPO_SHORT(64); break;
    }
#undef HIPO_SHORT
  } else if (const SharedMaskPlan sp = vec && rows < (int64_t{1} << 31)
                                            ? shared_mask_plan(batch, q, k, mask_batch_stride, heads)
                                            : SharedMaskPlan{};
             sp.k > 0) {
    if (sp.k == 1024) {
      launch_shared_mask<1024>(sp, stream, x, mask, out, batch, q, mask_row_stride,
                               mask_batch_stride, scale);
    } else {
      launch_shared_mask<2048>(sp, stream, x, mask, out, batch, q, mask_row_stride,
                               mask_batch_stride, scale);
    }
  } else if (vec) {
    const int64_t blocks = (rows + plan.rows_per_block - 1) / plan.rows_per_block;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "%s: too many rows", what);
    const dim3 grid(static_cast<unsigned>(blocks));
#define HIPO_SOFTMAX(U_, W_)                                                            \
  launch_vec<U_, W_>(grid, plan, stream, x, mask, out, rows, q, k, mask_row_stride,   \
                     mask_batch_stride, heads, scale)
    HIPO_ROW_DISPATCH(plan, HIPO_SOFTMAX);
#undef HIPO_SOFTMAX
  } else {
    const int64_t blocks = (rows + 3) / 4;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "%s: too many rows", what);
    masked_softmax_rows_scalar<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
        x, mask, out, rows, q, k, mask_row_stride, mask_batch_stride, heads, scale);
  }
  return check_launch(what);
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
  return hipo::softmax_impl(x, mask, out, batch, q, k, mask_row_stride, 0, 1, scale, stream,
                            "scaled_masked_softmax_bf16");
}

extern "C" int hipo_scaled_bias_softmax_bf16(const uint16_t* x, const uint16_t* bias,
                                             uint16_t* out, int64_t batch, int64_t q,
                                             int64_t k, int64_t bias_row_stride,
                                             int64_t bias_batch_stride, int64_t heads,
                                             float scale, hipStream_t stream) {
  return hipo::softmax_impl(x, bias, out, batch, q, k, bias_row_stride, bias_batch_stride,
                            heads, scale, stream, "scaled_bias_softmax_bf16");
}
