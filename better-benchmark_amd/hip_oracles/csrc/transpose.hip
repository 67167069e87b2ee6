// Batched transpose of the last two dimensions, bit for bit:
//   y[b, c, r] = x[b, r, c]     x: [batch, R, C], y: [batch, C, R], contiguous,
// for 2- and 4-byte elements (bf16 / fp16 / fp32 moved as bits).  This is
// permute(0, 1, 3, 2) + clone(contiguous_format) of a contiguous tensor.
//
// Whole matrices through LDS (R * C * size <= 32 KiB): a workgroup takes G
// consecutive matrices, which are one contiguous run of the input and one
// of the output.  It reads its input run with 16-byte non-temporal loads in
// memory order, scatters the elements into LDS in OUTPUT order, and writes
// its output run with 16-byte loads from LDS and 16-byte non-temporal
// stores in memory order -- both HBM streams are flat, whatever R and C
// are (R = 49 and 196 in the visformer attention-to-image layouts, whose
// output rows are not 16-byte multiples).  The LDS holds the output as
// 16-byte slots; in the scatter, consecutive lanes hold consecutive input
// vectors of one row, whose elements land R slots apart, so for even R a
// pad slot follows every R slots (slot q lives at q + q / R), making the
// lane stride R + 1 odd and the bank conflicts of the 2-byte LDS writes
// 4-way instead of 16-way or worse.
// Requires C * size % 16 == 0 and 16-byte aligned x, y for the vector
// loads; otherwise elements move one by one (same LDS scheme, no pad).
//
// Larger matrices: 64 x 64 tiles through LDS, one element per thread per
// step (coalesced 128- or 256-byte rows on both sides).
// HBM-bound: algorithmic bytes per element = 2 x size.
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kTrThreads = 256;
constexpr int kTrMaxBytes = 32 * 1024;          // data per workgroup (whole path)
constexpr int kTrMaxVecPerThread = kTrMaxBytes / 16 / kTrThreads;

struct WholeGeom {
  int64_t batch;
  int R, C, M;          // M = R * C elements per matrix
  int G;                // matrices per workgroup
  DivMagic by_m, by_c, by_r;
  bool pad;             // a pad slot after every R slots
};

template <typename T>
__device__ __forceinline__ T word_elem(const u32x4_t& v, int j) {
  if constexpr (sizeof(T) == 2) {
    return static_cast<T>((v[j >> 1] >> ((j & 1) * 16)) & 0xffffu);
  } else {
    return static_cast<T>(v[j]);
  }
}

// U: 16-byte input vectors per thread (VEC), the smallest power of two that
// covers the workgroup's run; 0 for the element path.
template <typename T, int U>
__global__ __launch_bounds__(kTrThreads) void transpose_whole(const T* __restrict__ x,
                                                              T* __restrict__ y, WholeGeom g) {
  extern __shared__ __align__(16) u32x4_t slots[];
  constexpr int V = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte slot
  T* lds = reinterpret_cast<T*>(slots);
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * g.G;
  const int gcount = static_cast<int>(g.batch - b0 < g.G ? g.batch - b0 : g.G);
  const int elems = gcount * g.M;
  const T* xb = x + b0 * g.M;
  T* yb = y + b0 * g.M;

  if constexpr (U > 0) {
    const int nvec = elems / V;
    const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(xb);
    // Straight-line code: every load is issued before the first is used.
    // Slots past the end take the last vector again and write the same
    // values to the same LDS places as its owner (no branch, no race: the
    // bits are identical).
    u32x4_t v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int iv = static_cast<int>(threadIdx.x) + k * kTrThreads;
      v[k] = __builtin_nontemporal_load(xv + (iv < nvec ? iv : nvec - 1));
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int iv0 = static_cast<int>(threadIdx.x) + k * kTrThreads;
      const int iv = iv0 < nvec ? iv0 : nvec - 1;
      // Input vector iv: matrix gi, row r, columns c0 .. c0 + V - 1 (one row);
      // output rows row0 .. row0 + V - 1 of the block, all in one pad group
      // (row0 is a multiple of V).
      const uint32_t f = static_cast<uint32_t>(iv) * V;
      const uint32_t gi = div_by(f, g.by_m);
      const uint32_t rem = f - gi * static_cast<uint32_t>(g.M);
      const uint32_t r = div_by(rem, g.by_c);
      const uint32_t c0 = rem - r * static_cast<uint32_t>(g.C);
      const uint32_t row0 = gi * static_cast<uint32_t>(g.C) + c0;
      const uint32_t e0 = row0 * static_cast<uint32_t>(g.R) + r + (g.pad ? row0 : 0u);
#pragma unroll
      for (int j = 0; j < V; ++j) lds[e0 + j * static_cast<uint32_t>(g.R)] = word_elem<T>(v[k], j);
    }
    __syncthreads();
    const int nslots = elems / V;
    u32x4_t* yv = reinterpret_cast<u32x4_t*>(yb);
    for (int o = threadIdx.x; o < nslots; o += kTrThreads) {
      const uint32_t s = static_cast<uint32_t>(o) +
                         (g.pad ? div_by(static_cast<uint32_t>(o), g.by_r) : 0u);
      __builtin_nontemporal_store(slots[s], yv + o);
    }
  } else {
    for (int f = threadIdx.x; f < elems; f += kTrThreads) {
      const uint32_t gi = div_by(static_cast<uint32_t>(f), g.by_m);
      const uint32_t rem = static_cast<uint32_t>(f) - gi * static_cast<uint32_t>(g.M);
      const uint32_t r = div_by(rem, g.by_c);
      const uint32_t c = rem - r * static_cast<uint32_t>(g.C);
      lds[(gi * static_cast<uint32_t>(g.C) + c) * static_cast<uint32_t>(g.R) + r] = xb[f];
    }
    __syncthreads();
    for (int f = threadIdx.x; f < elems; f += kTrThreads) yb[f] = lds[f];
  }
}

constexpr int kTile = 64;

// Any R, C: 64 x 64 tiles; grid = tiles of one matrix x batch, 1-D.
template <typename T>
__global__ __launch_bounds__(kTrThreads) void transpose_tiles(const T* __restrict__ x,
                                                              T* __restrict__ y, int64_t R,
                                                              int64_t C, int64_t r_tiles,
                                                              int64_t c_tiles) {
  __shared__ T tile[kTile][kTile + 1];
  const int64_t per_mat = r_tiles * c_tiles;
  const int64_t b = blockIdx.x / per_mat;
  const int64_t t = blockIdx.x % per_mat;
  const int64_t r0 = (t / c_tiles) * kTile;
  const int64_t c0 = (t % c_tiles) * kTile;
  const int tx = threadIdx.x & (kTile - 1);
  const int ty = threadIdx.x >> 6;
  const T* xm = x + b * R * C;
  T* ym = y + b * R * C;
  for (int i = ty; i < kTile; i += kTrThreads / kTile) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < R && c < C) tile[i][tx] = xm[r * C + c];
  }
  __syncthreads();
  for (int i = ty; i < kTile; i += kTrThreads / kTile) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (r < R && c < C) ym[c * R + r] = tile[tx][i];
  }
}

template <typename T>
int launch_transpose(const void* xp, void* yp, int64_t batch, int64_t R, int64_t C,
                     hipStream_t stream) {
  const T* x = static_cast<const T*>(xp);
  T* y = static_cast<T*>(yp);
  constexpr int V = 16 / static_cast<int>(sizeof(T));
  const int64_t mat_bytes = R * C * static_cast<int64_t>(sizeof(T));
  if (mat_bytes <= kTrMaxBytes) {
    WholeGeom g;
    g.batch = batch;
    g.R = static_cast<int>(R);
    g.C = static_cast<int>(C);
    g.M = static_cast<int>(R * C);
    // Several small matrices per workgroup only when that still leaves
    // over a thousand workgroups.
    int64_t G = kTrMaxBytes / mat_bytes;
    const int64_t spread = batch / 1024 > 1 ? batch / 1024 : 1;
    if (G > spread) G = spread;
    g.G = static_cast<int>(G);
    g.by_m = div_magic(static_cast<uint32_t>(g.M));
    g.by_c = div_magic(static_cast<uint32_t>(g.C));
    g.by_r = div_magic(static_cast<uint32_t>(g.R));
    const bool vec = (C * static_cast<int64_t>(sizeof(T))) % 16 == 0 && aligned16(x) &&
                     aligned16(y);
    g.pad = vec && R % 2 == 0;
    const int64_t slots_used = G * g.M / V;
    const int64_t pads = g.pad ? slots_used / R + 1 : 0;
    const size_t lds_bytes =
        vec ? static_cast<size_t>(slots_used + pads) * 16
            : static_cast<size_t>(G * g.M) * sizeof(T);
    const int64_t blocks = (batch + G - 1) / G;
    HIPO_REQUIRE(blocks < (int64_t{1} << 31), "transpose: too many matrices");
    const dim3 grid(static_cast<unsigned>(blocks)), block(kTrThreads);
    const int64_t per_thread = (slots_used + kTrThreads - 1) / kTrThreads;
    if (!vec) {
      transpose_whole<T, 0><<<grid, block, lds_bytes, stream>>>(x, y, g);
    } else if (per_thread <= 1) {
      transpose_whole<T, 1><<<grid, block, lds_bytes, stream>>>(x, y, g);
    } else if (per_thread <= 2) {
      transpose_whole<T, 2><<<grid, block, lds_bytes, stream>>>(x, y, g);
    } else if (per_thread <= 4) {
      transpose_whole<T, 4><<<grid, block, lds_bytes, stream>>>(x, y, g);
    } else {
      transpose_whole<T, kTrMaxVecPerThread><<<grid, block, lds_bytes, stream>>>(x, y, g);
    }
  } else {
    const int64_t r_tiles = (R + kTile - 1) / kTile;
    const int64_t c_tiles = (C + kTile - 1) / kTile;
    const int64_t blocks = batch * r_tiles * c_tiles;
    HIPO_REQUIRE(blocks < (int64_t{1} << 31), "transpose: too many tiles");
    transpose_tiles<T><<<dim3(static_cast<unsigned>(blocks)), dim3(kTrThreads), 0, stream>>>(
        x, y, R, C, r_tiles, c_tiles);
  }
  return 0;
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_transpose_last2(const void* x, void* y, int64_t batch, int64_t rows,
                                    int64_t cols, int elem_size, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0, "transpose: negative size");
  HIPO_REQUIRE(elem_size == 2 || elem_size == 4,
               "transpose: element size %d (2 or 4 bytes supported)", elem_size);
  if (batch == 0 || rows == 0 || cols == 0) return 0;
  HIPO_REQUIRE(x && y, "transpose: null pointer");
  HIPO_REQUIRE(x != y, "transpose: x and y must not alias");
  HIPO_REQUIRE(rows <= 0x7fffffff && cols <= 0x7fffffff, "transpose: dimension too large");
  const int rc = elem_size == 2 ? launch_transpose<uint16_t>(x, y, batch, rows, cols, stream)
                                : launch_transpose<uint32_t>(x, y, batch, rows, cols, stream);
  if (rc != 0) return rc;
  return check_launch("transpose_last2");
}
