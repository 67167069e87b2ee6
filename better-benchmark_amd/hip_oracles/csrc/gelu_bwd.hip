// GELU (erf form) backward fused with the column sum of its output, bf16:
//   y[r, c]    = bf16(g[r, c] * d(x[r, c]))
//   d(t)       = Phi(t) + t phi(t) = 0.5 (1 + erf(t / sqrt 2)) + t exp(-t^2 / 2) / sqrt(2 pi)
//   colsum[c]  = bf16(sum_r y[r, c]), stored as fp32
// -- the graph of the reference's sum_139a3020e8bf (timm / HF training: the
// gradient through an erf GELU and its bias gradient).
//
// d is a function of a bf16 input, so it is read, not computed: the kernel
// stages a 32 KiB table of the correctly rounded fp32 d(t) of every bf16 t
// (gelu_grad_table.h, 2 signs x 32 exponent rows x 128 mantissas; exponents
// clamped to the rows whose values differ) into LDS and multiplies g by the
// entry -- one fp32 product and one rounding to bf16 per element, about a
// dozen VALU operations with the indexing, where evaluating erf and exp costs
// about 56 and makes the kernel VALU-bound at large shapes.  inf and NaN
// inputs give NaN (t * 0 added to the entry).  Eager evaluates the graph's
// chain of fp32 operations, whose 1 + erf cancels for negative t; its d is
// within a few fp32 ulps of this one, so single y elements can differ from
// eager's by one bf16 ulp at rounding boundaries, this side being the
// correctly rounded product.
//
// The column sums are fp64 throughout (per lane, over the waves, over the
// row blocks): a sum of bf16 values in fp64 is exact unless its terms span
// more than about 53 - 8 - log2(rows) binades, so colsum is the correctly
// rounded bf16 of the exact sum, whatever the order -- an fp32 sum rounded
// to bf16 lands on the wrong side of a bf16 rounding boundary now and then
// when its order differs from another's.
//
// Layout: a workgroup of 4 or 16 waves takes a block of rows x 512 columns
// (64 lanes x one 16-byte group of 8 bf16); wave w handles rows w, w + W,
// ... of the block, two rows' loads issued together, so per row a wave reads
// 1 KiB of g and of x and writes 1 KiB of y (non-temporal).  Every load and
// store is unconditional -- a lane past the last column group, or a wave
// past the block's last row, re-addresses the last group / row and stores
// the bytes its owner stores -- so the compiler's wait counts stay exact;
// only the column sums are guarded.  The workgroup's per-lane sums are
// merged over its waves in LDS and written as one row of fp64 partial sums
// per (row block, column block); a second kernel adds each column's partials
// (a fixed tree) and rounds once (fp64 -> bf16) to nearest even.
// Up to 256 rows a single kernel does both (gelu_erf_bwd_small below).
// Measured on MI355X against whole-row workgroups (all of a row's column
// blocks in one workgroup) and loops that prefetch the next rows, this is
// the fastest layout tried: 0.7-0.8 of a flat copy of the same three
// streams at the large shapes.
// Bytes: 4 read + 2 written per element, plus 16 per column and row block
// for the partials and 32 KiB of table per workgroup (from L2).
#include "gelu_grad_table.h"
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kColBlock = kWave * 8;   // 512 columns per workgroup
constexpr int kRows = 2;               // rows per wave whose loads go out together
constexpr int64_t kSmallRows = 256;    // up to here: the one-launch kernel

// d(t) for the bf16 input with bits hb (low 16 bits), as a table index.  The
// magnitude bits (exponent and mantissa) are clamped to the table's rows as
// a whole: the first and last rows are constant, so any mantissa of a
// clamped exponent reads the same value.
constexpr uint32_t kMagLo = kGeluGradExpLo << 7;
constexpr uint32_t kMagHi = (kGeluGradExpHi << 7) | 0x7fu;

__device__ __forceinline__ uint32_t lut_index(uint32_t hb) {
  const uint32_t mag =
      __builtin_elementwise_min(__builtin_elementwise_max(hb & 0x7fffu, kMagLo), kMagHi);
  return ((hb >> 15) & 1u) * static_cast<uint32_t>(kGeluGradPerSign) + mag - kMagLo;
}

// One row group of 8 elements: the 8 indices, the 8 table reads together,
// then the products (t * 0 + d: NaN for inf and NaN t).
__device__ __forceinline__ u32x4_t row_grad(const u32x4_t& gv, const u32x4_t& xv,
                                            const float* lut) {
  uint32_t idx[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    idx[2 * d] = lut_index(xv[d] & 0xffffu);
    idx[2 * d + 1] = lut_index(xv[d] >> 16);
  }
  float dv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dv[e] = lut[idx[e]];
  u32x4_t o;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    o[d] = pack_bf16x2(bf16lo(gv[d]) * __builtin_fmaf(bf16lo(xv[d]), 0.0f, dv[2 * d]),
                       bf16hi(gv[d]) * __builtin_fmaf(bf16hi(xv[d]), 0.0f, dv[2 * d + 1]));
  return o;
}

// The bf16 nearest to the fp64 s (ties to even), as an fp32 value, with one
// rounding: hi = fp32(s) can only sit on the wrong side of a bf16 rounding
// boundary when it is that boundary, and then the sign of s - hi decides.
__device__ __forceinline__ float bf16_of_f64(double s) {
  const float hi = static_cast<float>(s);
  const double lo = s - static_cast<double>(hi);
  const uint32_t b = __float_as_uint(hi);
  if ((b & 0xffffu) == 0x8000u && lo != 0.0) {
    const bool away = (lo > 0.0) == (hi > 0.0f);  // |s| above the midpoint
    return __uint_as_float(away ? (b + 0x8000u) & 0xffff0000u : b & 0xffff0000u);
  }
  return round_bf16(hi);
}

template <int kThreads>
constexpr int tile_lds_floats() {
  // the table, then each wave's 8 fp64 sums per lane
  return kGeluGradTableSize > kThreads * 16 ? kGeluGradTableSize : kThreads * 16;
}

// grid: x = column block, y = row block.
template <int kThreads>
__global__ __launch_bounds__(kThreads) void gelu_erf_bwd_tiles(
    const uint16_t* __restrict__ g, const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
    double* __restrict__ partial, int64_t rows, int cols, int64_t rows_per_block) {
  constexpr int kWaves = kThreads / kWave;
  __shared__ __align__(16) float lds[tile_lds_floats<kThreads>()];
  for (int i = threadIdx.x; i < kGeluGradTableSize / 4; i += kThreads)
    reinterpret_cast<u32x4_t*>(lds)[i] = reinterpret_cast<const u32x4_t*>(kGeluGradTable)[i];
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int col = static_cast<int>(blockIdx.x) * kColBlock + lane * 8;
  const bool col_ok = col < cols;
  const int colc = col_ok ? col : cols - 8;  // the last group: same bytes as its owner
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;

  double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  for (int64_t rb = r0 + wave; rb < r1; rb += static_cast<int64_t>(kWaves) * kRows) {
    u32x4_t gv[kRows], xv[kRows];
#pragma unroll
    for (int f = 0; f < kRows; ++f) {
      const int64_t r = rb + static_cast<int64_t>(f) * kWaves;
      const int64_t off = (r < r1 ? r : r1 - 1) * cols + colc;
      gv[f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(g + off));
      xv[f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + off));
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads out before the first use
#pragma unroll
    for (int f = 0; f < kRows; ++f) {
      const int64_t r = rb + static_cast<int64_t>(f) * kWaves;  // wave-uniform
      const u32x4_t o = row_grad(gv[f], xv[f], lds);
      __builtin_nontemporal_store(
          o, reinterpret_cast<u32x4_t*>(y + (r < r1 ? r : r1 - 1) * cols + colc));
      if (r < r1) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          acc[2 * d] += bf16lo(o[d]);
          acc[2 * d + 1] += bf16hi(o[d]);
        }
      }
    }
  }

  __syncthreads();  // the table is dead: its LDS holds the waves' sums now
  double* red = reinterpret_cast<double*>(lds);
#pragma unroll
  for (int e = 0; e < 8; ++e) red[(wave * 8 + e) * kWave + lane] = acc[e];
  __syncthreads();
  if (wave == 0 && col_ok) {
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += red[(w * 8 + e) * kWave + lane];
    }
    double* dst = partial + static_cast<int64_t>(blockIdx.y) * cols + col;
#pragma unroll
    for (int e = 0; e < 8; e += 2)
      *reinterpret_cast<double2*>(dst + e) = double2{acc[e], acc[e + 1]};
  }
}

// Up to 256 rows: one launch, no workspace.  A workgroup of 16 waves owns 64
// columns of every row: lane = 8 * column group + row, so a wave covers 8
// rows x 64 columns (8 x 128 contiguous bytes per tensor) and the
// workgroup 128 rows per pass, kPasses passes' loads issued before the
// table is staged (the two latencies overlap).  Column sums: fp64 per lane,
// over a wave's 8 rows with DPP butterflies (sum8), over the 16 waves in
// order through LDS, then one rounding to bf16 -- the same value as the
// two-kernel path's.
template <int kPasses>
__global__ __launch_bounds__(1024) void gelu_erf_bwd_small(
    const uint16_t* __restrict__ g, const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
    float* __restrict__ colsum, int rows, int cols) {
  constexpr int kSmallWaves = 16;
  __shared__ __align__(16) float lds[kGeluGradTableSize];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int cg = lane >> 3;
  const int rl = lane & 7;
  const int col = static_cast<int>(blockIdx.x) * 64 + cg * 8;
  const int colc = col < cols ? col : cols - 8;  // the last group: same bytes as its owner
  u32x4_t gv[kPasses], xv[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int r = p * 8 * kSmallWaves + wave * 8 + rl;
    const int64_t off = static_cast<int64_t>(r < rows ? r : rows - 1) * cols + colc;
    gv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(g + off));
    xv[p] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + off));
  }
  for (int i = threadIdx.x; i < kGeluGradTableSize / 4; i += 1024)
    reinterpret_cast<u32x4_t*>(lds)[i] = reinterpret_cast<const u32x4_t*>(kGeluGradTable)[i];
  __syncthreads();
  double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int r = p * 8 * kSmallWaves + wave * 8 + rl;
    const u32x4_t o = row_grad(gv[p], xv[p], lds);
    __builtin_nontemporal_store(
        o, reinterpret_cast<u32x4_t*>(y + static_cast<int64_t>(r < rows ? r : rows - 1) * cols +
                                      colc));
    const bool ok = r < rows;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc[2 * d] += ok ? static_cast<double>(bf16lo(o[d])) : 0.0;
      acc[2 * d + 1] += ok ? static_cast<double>(bf16hi(o[d])) : 0.0;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = sum8(acc[e]);  // over the wave's 8 rows
  __syncthreads();  // the table is dead: its LDS holds the waves' sums now
  double* red = reinterpret_cast<double*>(lds);
  if (rl == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[(wave * 8 + cg) * 8 + e] = acc[e];
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int c = static_cast<int>(blockIdx.x) * 64 + static_cast<int>(threadIdx.x);
    double t = red[threadIdx.x];
#pragma unroll
    for (int w = 1; w < kSmallWaves; ++w) t += red[w * 64 + threadIdx.x];
    if (c < cols) colsum[c] = bf16_of_f64(t);
  }
}

// colsum[c] = bf16(sum over row blocks of partial[rb][c]), stored as fp32.
// A workgroup of 256 threads takes kCols columns (thread % kCols) and splits
// the row blocks over 256 / kCols slices (slice j: j, j + S, ...; 8 loads in
// flight), then adds the slices in a fixed tree.  kCols is picked so that
// narrow tensors still spread over a few hundred workgroups.  With no row
// blocks it writes zeros.
constexpr int kFinishThreads = 256;

template <int kCols>
__global__ __launch_bounds__(kFinishThreads) void colsum_finish(const double* __restrict__ partial,
                                                                float* __restrict__ colsum,
                                                                int row_blocks, int cols) {
  constexpr int kSlices = kFinishThreads / kCols;
  const int l = threadIdx.x % kCols;
  const int j = threadIdx.x / kCols;
  // XCD-aware order: workgroup ids go round-robin over the 8 XCDs; each XCD
  // takes a contiguous range of column groups, so the partial rows' cache
  // lines, which kCols-column groups share, are fetched into one L2.  (After
  // a cache flush, [175360, 3072] / [25216, 3072]: 569 -> 557 / 97.6 -> 94.4
  // us for the whole call.)
  const int nb = static_cast<int>(gridDim.x);
  const int bid = static_cast<int>(blockIdx.x);
  const int grp = nb % 8 == 0 ? (bid % 8) * (nb / 8) + bid / 8 : bid;
  const int c = grp * kCols + l;
  const bool ok = c < cols;
  const int cc = ok ? c : cols - 1;
  double s = 0.0;
  constexpr int kUnroll = 8;
  for (int rb = j; rb < row_blocks; rb += kSlices * kUnroll) {
    double v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int k = rb + u * kSlices;
      v[u] = k < row_blocks ? partial[static_cast<int64_t>(k) * cols + cc] : 0.0;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) s += v[u];
  }
  __shared__ double part[kFinishThreads];
  part[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int half = kSlices / 2; half > 0; half /= 2) {  // slice j += slice j + half
    if (j < half) part[threadIdx.x] += part[threadIdx.x + half * kCols];
    __syncthreads();
  }
  if (j == 0 && ok) colsum[c] = bf16_of_f64(part[l]);
}

// Columns per finishing workgroup: about cols / 512 (so ~512 workgroups),
// a power of two in [1, 64].
int finish_cols(int64_t cols) {
  int k = 1;
  while (k < 64 && static_cast<int64_t>(k) * 2 * 512 <= cols) k *= 2;
  return k;
}

int launch_finish(const double* partial, float* colsum, int row_blocks, int64_t cols,
                  hipStream_t stream) {
  const int k = finish_cols(cols);
  const dim3 grid(static_cast<unsigned>((cols + k - 1) / k));
  const int c = static_cast<int>(cols);
  switch (k) {
    case 1: colsum_finish<1><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
    case 2: colsum_finish<2><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
    case 4: colsum_finish<4><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
    case 8: colsum_finish<8><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
    case 16: colsum_finish<16><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
    case 32: colsum_finish<32><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
    default: colsum_finish<64><<<grid, kFinishThreads, 0, stream>>>(partial, colsum, row_blocks, c); break;
  }
  return check_launch("gelu_erf_bwd_colsum_bf16");
}

struct BwdPlan {
  int threads = 0;
  int col_blocks = 0;
  int row_blocks = 0;
  int64_t rows_per_block = 0;
};

// Measured on MI355X over the corpus shapes (256 to 1024 threads, 256 to
// 8192 workgroups): 16-wave workgroups, with rows per block set by width --
// one or two column blocks want long blocks (256 rows: few partial rows for
// the finishing pass to read), wider tensors about rows * col_blocks / 2048
// rows (some 2000 workgroups), held to [64, 128] up to 8 column blocks and
// [32, 128] beyond.  From 257 to 1024 rows: 4-wave workgroups of 8 rows,
// the most workgroups for a small launch.
BwdPlan bwd_plan(int64_t rows, int64_t cols) {
  BwdPlan p;
  p.col_blocks = static_cast<int>((cols + kColBlock - 1) / kColBlock);
  int64_t rpb;
  if (rows <= 1024) {
    p.threads = 256;
    rpb = 8;
  } else {
    p.threads = 1024;
    if (p.col_blocks <= 2) {
      // Long blocks, halved while they would leave most CUs idle (fewer
      // than 192 workgroups): [8192, 768] 23.5 -> 13.6 us back to back with
      // 64-row blocks (256 workgroups) instead of 256-row ones (64); at
      // [25216, 768] and [32768, 1024] (198 and 256 workgroups of 256 rows)
      // shorter blocks were 1-8 % slower.
      rpb = 256;
      while (rpb > 32 && (rows + rpb - 1) / rpb * p.col_blocks < 192) rpb /= 2;
    } else {
      const int64_t lo = p.col_blocks <= 8 ? 64 : 32;
      rpb = rows * p.col_blocks / 2048;
      rpb = rpb < lo ? lo : rpb > 128 ? 128 : rpb;
    }
  }
  constexpr int64_t kMaxRowBlocks = 65535;  // grid.y
  if ((rows + rpb - 1) / rpb > kMaxRowBlocks) rpb = (rows + kMaxRowBlocks - 1) / kMaxRowBlocks;
  p.rows_per_block = rpb;
  p.row_blocks = static_cast<int>((rows + rpb - 1) / rpb);
  return p;
}

}  // namespace
}  // namespace hipo

extern "C" size_t hipo_gelu_erf_bwd_colsum_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= hipo::kSmallRows || cols <= 0 || cols > 0x7fffffff) return 0;
  const hipo::BwdPlan p = hipo::bwd_plan(rows, cols);
  return static_cast<size_t>(p.row_blocks) * static_cast<size_t>(cols) * sizeof(double);
}

extern "C" int hipo_gelu_erf_bwd_colsum_bf16(const uint16_t* grad, const uint16_t* x,
                                             uint16_t* y, float* colsum, int64_t rows,
                                             int64_t cols, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(rows >= 0 && cols >= 0, "gelu_erf_bwd: negative size");
  if (cols == 0) return 0;
  HIPO_REQUIRE(cols % 8 == 0 && cols <= 0x7fffffff,
               "gelu_erf_bwd: cols must be a multiple of 8 (got %lld)", (long long)cols);
  HIPO_REQUIRE(colsum != nullptr, "gelu_erf_bwd: null colsum");
  if (rows == 0)  // colsum = 0 by the finishing kernel (no memset: capture-safe)
    return launch_finish(nullptr, colsum, 0, cols, stream);
  HIPO_REQUIRE(grad && x && y, "gelu_erf_bwd: null pointer");
  HIPO_REQUIRE(aligned16(grad) && aligned16(x) && aligned16(y),
               "gelu_erf_bwd: grad, x and y must be 16-byte aligned");
  const int c = static_cast<int>(cols);
  if (rows <= kSmallRows) {
    const dim3 grid(static_cast<unsigned>((cols + 63) / 64));
    const int r = static_cast<int>(rows);
    if (rows <= kSmallRows / 2)
      gelu_erf_bwd_small<1><<<grid, 1024, 0, stream>>>(grad, x, y, colsum, r, c);
    else
      gelu_erf_bwd_small<2><<<grid, 1024, 0, stream>>>(grad, x, y, colsum, r, c);
    return check_launch("gelu_erf_bwd_colsum_bf16");
  }
  HIPO_REQUIRE(workspace && aligned16(workspace),
               "gelu_erf_bwd: workspace must be non-null and 16-byte aligned");
  const BwdPlan p = bwd_plan(rows, cols);
  const size_t need =
      static_cast<size_t>(p.row_blocks) * static_cast<size_t>(cols) * sizeof(double);
  HIPO_REQUIRE(workspace_bytes >= need, "gelu_erf_bwd: workspace of %zu bytes, need %zu",
               workspace_bytes, need);
  const dim3 grid(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.row_blocks));
  double* partial = static_cast<double*>(workspace);
  if (p.threads == 1024)
    gelu_erf_bwd_tiles<1024><<<grid, 1024, 0, stream>>>(grad, x, y, partial, rows, c,
                                                        p.rows_per_block);
  else
    gelu_erf_bwd_tiles<256><<<grid, 256, 0, stream>>>(grad, x, y, partial, rows, c,
                                                      p.rows_per_block);
  const int rc = check_launch("gelu_erf_bwd_colsum_bf16");
  if (rc != 0) return rc;
  return launch_finish(partial, colsum, p.row_blocks, cols, stream);
}
