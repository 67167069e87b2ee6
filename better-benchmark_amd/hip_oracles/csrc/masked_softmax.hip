// Scaled, additively masked softmax over the last dim, bf16 in / bf16 out.
//
// Semantics (softmax(x * scale + mask, -1) on bf16, scores formed in fp32
// as the reference's Triton oracles and Inductor form them):
//   s = fma(x, scale, mask[q, :])                  (fp32, one rounding)
//   out = bf16(exp(s - max(s)) / sum(exp(s - max(s))))   (fp32 max and sum;
//         the quotient is the IEEE fp32 division's, div_rn)
// exp is natural exp of the fp32 difference s - max(s) (as aten.exp and
// Inductor's libdevice.exp), evaluated to about one ulp by exp_f32_nonpos,
// an extended-precision (Cody-Waite) reduction as the device library's
// (no exp2 rewrite).  Eager
// rounds x * scale and the sum to bf16 first; with a power-of-two scale and
// a 0 / -inf mask (the causal softmax) both roundings are exact, so the
// scores are eager's; with a general bias (TrOCR) the fp32 scores are the
// reference oracle's (its oracle.py builds them from fp32 x + bias) and
// several times closer to fp64 than eager's rounded ones.
//
// Layout: rows held in registers, non-temporal 16-byte streaming accesses
// for x and out; the mask row (mask[q, :], q = row % Q) is re-read by every
// batch entry and stays cache-resident.  Row max and row sum: DPP within a
// wave, then (where a row spans several waves) a fixed-order combine of the
// wave results through LDS.  Three
// kernels by row length:
//   K <= 512: L lanes per row, 64 / L rows per access instruction, 2 KiB of
//     x per wave, reductions within lane segments, no LDS;
//   K = 1024 or 2048 (config [384, 1024, 1024]): one wave per row (2 or 4
//     KiB of x), the rows of one q for 4 consecutive batch entries in a
//     256-thread workgroup, their shared mask row loaded once and staged
//     through LDS, row reductions within the wave;
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
  // s - m <= 0 (m is the row max) or NaN, so only the lower bound needs
  // the clamp (IEEE maximum: NaN stays NaN).
  return exp_f32_nonpos(__builtin_elementwise_maximum(s - m, -104.0f));
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
#pragma unroll
    for (int d = 0; d < 4; ++d)
      o[d] = pack_bf16x2(div_rn(s[u][2 * d], sum, inv), div_rn(s[u][2 * d + 1], sum, inv));
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
    const float tot = seg_sum<L>(sum);
    const float inv = 1.0f / tot;
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      o[d] = pack_bf16x2(div_rn(s[2 * d], tot, inv), div_rn(s[2 * d + 1], tot, inv));
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

// Rows of exactly K = 1024 or 2048 (KC, a compile-time constant): whole
// rows per wave, the shared mask row staged once per workgroup.  Workgroup
// (q, y, z) of the 3-D grid takes the NW * RPW rows (b0 + wave + NW i) * Q +
// q, b0 = (z * gy + y) * NW * RPW: the same q of consecutive batch entries,
// which share mask[q, :]; z is the mask's batch group (offset z *
// mask_batch_stride; a single z when the mask is broadcast over batch) and
// gy its workgroups along y, so the kernel does no integer division; x is
// fastest, so dispatch order walks q in memory order.  Each wave owns its
// RPW rows entirely -- G = KC / 512 16-byte groups per lane per row, group g
// covering columns [512 g, 512 g + 512) across the wave -- so a row's max
// and sum are wave reductions with no LDS exchange, and the only barrier is
// the mask staging (the row's 2 KC bytes, loaded before the x rows).  A
// column group whose 512 scores are all -inf in a row (the causal upper
// triangle: group 1 of every row q < 512 at K = 1024) skips its exp.  Rows
// past the batch end re-read the last batch entry and store nothing.
// Measured at [384, 1024, 1024] (steady loop, same process; a flat copy of
// the same bytes 246.9-247.5 us): 4 waves x 1 row (shipped) 252.9-254.6 us;
// 4 x 2 rows 258.3-259.9; 4 x 4 rows 270.7; 2 / 8 waves x 1 row 257.3-258.2
// / 258.5-258.8; the previous layout (2 waves per row, 1 KiB each, 4 rows
// per wave, maxima and sums exchanged through LDS) 258.0-261.8; 8
// consecutive rows of one batch entry per workgroup, each wave reading its
// mask rows through the cache, 274.2-275.7.  Timing probes of the 4 x 2
// layout with the exp replaced by a bare exp2, or removed, or without the
// division correction, all ran 258-260 us: these rows are bound by their
// memory pattern, not by arithmetic.
template <int KC, int NW, int RPW>
__global__ __launch_bounds__(NW * 64) void masked_softmax_wave_rows(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ mask,
    uint16_t* __restrict__ out, uint32_t batch, uint32_t Q, uint32_t gy,
    int64_t mask_stride, int64_t mask_batch_stride, float scale) {
  constexpr int G = KC / 512;
  constexpr int kThreads = NW * kWave;
  constexpr int kStageWords = KC / 2 / kThreads;  // 32-bit mask words per thread
  static_assert(kStageWords * kThreads * 2 == KC, "the mask row splits evenly");
  __shared__ __align__(16) uint32_t mrow[KC / 2];  // read back as 16-byte groups
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const uint32_t q = blockIdx.x;
  const uint32_t b0 = (blockIdx.z * gy + blockIdx.y) * (NW * RPW) + wave;

  const uint32_t* mr = reinterpret_cast<const uint32_t*>(
      mask + blockIdx.z * mask_batch_stride + static_cast<int64_t>(q) * mask_stride);
  uint32_t mval[kStageWords];
#pragma unroll
  for (int k = 0; k < kStageWords; ++k) mval[k] = mr[threadIdx.x + k * kThreads];
  u32x4_t xv[RPW][G];
  int64_t row[RPW];
  bool row_ok[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const uint32_t b = b0 + NW * i;
    row_ok[i] = b < batch;
    // Rows past the batch end re-read the last batch entry and store nothing.
    row[i] = static_cast<int64_t>(row_ok[i] ? b : batch - 1) * Q + q;
#pragma unroll
    for (int g = 0; g < G; ++g)
      xv[i][g] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(x + row[i] * KC + g * 512 + lane * kRowGroup));
  }
#pragma unroll
  for (int k = 0; k < kStageWords; ++k) mrow[threadIdx.x + k * kThreads] = mval[k];
  __syncthreads();
  u32x4_t mv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    mv[g] = *reinterpret_cast<const u32x4_t*>(&mrow[(g * 512 + lane * kRowGroup) / 2]);

#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    float sc[G][8];
    float gmax[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      gmax[g] = -__builtin_inff();  // NaN-propagating: NaN if any score is
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        sc[g][2 * d] = __builtin_fmaf(bf16lo(xv[i][g][d]), scale, bf16lo(mv[g][d]));
        sc[g][2 * d + 1] = __builtin_fmaf(bf16hi(xv[i][g][d]), scale, bf16hi(mv[g][d]));
        gmax[g] = __builtin_elementwise_maximum(
            gmax[g], __builtin_elementwise_maximum(sc[g][2 * d], sc[g][2 * d + 1]));
      }
    }
    float lmax = gmax[0];
#pragma unroll
    for (int g = 1; g < G; ++g) lmax = __builtin_elementwise_maximum(lmax, gmax[g]);
    const float m = wave_maximum(lmax);
    // A column group that is -inf in every lane skips its exp (wave-
    // uniform); a lane of -inf scores in a live group gets exp = 0 from the
    // clamped argument; a NaN score keeps its group live, so the NaN reaches
    // the row sum, as in eager.
    bool live[G];
    float sum = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      live[g] = __builtin_amdgcn_ballot_w64(!(gmax[g] == -__builtin_inff())) != 0;
      if (live[g]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[g][e] = exp_shifted(sc[g][e], m);
        sum += ((sc[g][0] + sc[g][1]) + (sc[g][2] + sc[g][3])) +
               ((sc[g][4] + sc[g][5]) + (sc[g][6] + sc[g][7]));
      }
    }
    const float tot = wave_sum(sum);
    const float inv = 1.0f / tot;
    // p = e / sum, the IEEE quotient (div_rn), rounded to bf16.  A skipped
    // group's outputs are 0 * (1 / sum): 0, or NaN for a row whose every
    // score is -inf (sum 0), as in eager.
#pragma unroll
    for (int g = 0; g < G; ++g) {
      u32x4_t o;
      if (live[g]) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          o[d] = pack_bf16x2(div_rn(sc[g][2 * d], tot, inv), div_rn(sc[g][2 * d + 1], tot, inv));
      } else {
        const uint32_t z = pack_bf16x2(0.f * inv, 0.f * inv);
        o = u32x4_t{z, z, z, z};
      }
      if (row_ok[i])
        __builtin_nontemporal_store(
            o, reinterpret_cast<u32x4_t*>(out + row[i] * KC + g * 512 + lane * kRowGroup));
    }
  }
}

// Waves per workgroup and rows per wave of the whole-row kernel (a
// workgroup's rows: one query q of NW * RPW consecutive batch entries).
constexpr int kSharedMaskWaves = 4;
constexpr int kSharedMaskRowsPerWave = 1;

// Launch shape of the whole-row kernel: its row length (1024 or 2048; 0
// when the kernel does not apply) and the 3-D grid.  It does not apply to
// other K, to a per-batch mask whose heads groups the NW * RPW rows of a
// workgroup do not divide, or to grids beyond the y / z limits.
struct SharedMaskPlan {
  int k = 0;
  uint32_t gy = 0;  // workgroups along y per mask batch group
  dim3 grid;
};

SharedMaskPlan shared_mask_plan(int64_t batch, int64_t Q, int64_t K, int64_t mbs,
                                int64_t heads) {
  SharedMaskPlan plan;
  if ((K != 1024 && K != 2048) || Q > 0x7fffffff) return plan;
  const int nr = kSharedMaskWaves * kSharedMaskRowsPerWave;  // rows per workgroup
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
  masked_softmax_wave_rows<KC, kSharedMaskWaves, kSharedMaskRowsPerWave>
      <<<plan.grid, dim3(kSharedMaskWaves * kWave), 0, stream>>>(
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
    orow[j] = static_cast<uint16_t>(pack_bf16x2(div_rn(e, sum, inv), 0.f) & 0xffffu);
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
