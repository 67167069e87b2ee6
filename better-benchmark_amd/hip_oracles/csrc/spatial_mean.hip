// Spatial mean of a channels-last bf16 tensor: the reduction over a
// non-innermost axis.
//   x: [N, C, H, W] bf16 stored channels-last (physical [N, P, C], P = H*W)
//   out[n, c] = bf16(sum_p x[n, p, c] / P)          (fp32 accumulation)
// (torch.mean(x, [2, 3], keepdim) of the reference's mean_c9e1a8113328.)
//
// Layout.  G = C / 8 channel groups of 16 bytes (or a block of 64 of them,
// see spatial_plan).  A workgroup of T threads (T a multiple of G) reduces
// the positions [p0, p1) of one image: thread t
// owns group t % G and positions p0 + t / G + k * (T / G), so each load
// instruction of the workgroup covers T / G rows -- whole rows (T * 16
// contiguous bytes), or each row's 1 KiB of the channel block -- and each
// thread keeps 4 loads in flight.  The T / G partial sums of
// a group meet in LDS and the first G threads add them in a fixed order.
// With one position slice per image the result is written as bf16 directly;
// with S > 1 slices (more workgroups than images alone give) each slice
// writes fp32 partials and a second kernel adds the S slices of a channel in
// a fixed order.  Small images (at most 224 positions, C a multiple of 64,
// enough images) take spatial_mean_small_waves instead: one wave per (image,
// 64-channel block), every position in flight.  Deterministic.
// HBM-bound: algorithmic bytes = 2 N P C (read) + 2 N C (write).
#include <algorithm>

#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kUnroll = 4;
constexpr int kMaxThreads = 1024;

__global__ __launch_bounds__(kMaxThreads) void spatial_mean_nhwc_partial(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ out,
    float* __restrict__ partial, int64_t P, int64_t C, int G, int cblocks, int slices,
    int64_t slice_len) {
  extern __shared__ float lds[];  // [T][8]
  const int T = blockDim.x;
  const int t = threadIdx.x;
  const int gl = t % G;       // group within the workgroup's channel block
  const int r = t / G;        // row offset of this thread
  const int R = T / G;        // rows per workgroup instruction
  const int64_t n = blockIdx.x / (cblocks * slices);
  const int rest = blockIdx.x - static_cast<int>(n) * cblocks * slices;
  const int cb = rest / slices;
  const int s = rest - cb * slices;
  const int g = cb * G + gl;  // group within the row
  const int64_t p0 = s * slice_len;
  const int64_t p1 = std::min<int64_t>(P, p0 + slice_len);
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x + n * P * C) + g;
  const int64_t G64 = C / 8;  // groups per row

  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t p = p0 + r; p < p1; p += static_cast<int64_t>(R) * kUnroll) {
    u32x4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      // Positions past the slice re-read the slice's first row (in bounds)
      // and are zeroed.
      const int64_t pu = p + static_cast<int64_t>(u) * R;
      v[u] = __builtin_nontemporal_load(xv + (pu < p1 ? pu : p0) * G64);
      if (pu >= p1) v[u] = u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        acc[2 * d] += bf16lo(v[u][d]);
        acc[2 * d + 1] += bf16hi(v[u][d]);
      }
    }
  }
  if (R > 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) lds[t * 8 + e] = acc[e];
    __syncthreads();
    if (t < G) {
      for (int k = 1; k < R; ++k) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += lds[(k * G + t) * 8 + e];
      }
    }
  }
  if (t >= G) return;  // t == gl from here on
  if (slices == 1) {
    const float inv = 1.0f / static_cast<float>(P);
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = pack_bf16x2(acc[2 * d] * inv, acc[2 * d + 1] * inv);
    *reinterpret_cast<u32x4_t*>(out + n * C + 8 * g) = o;
  } else {
    float* dst = partial + (n * slices + s) * C + 8 * g;
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e] = acc[e];
  }
}

// Small images (spatial_small_plan): one wave per (image, block of 64
// channels), every position of the image in flight at once.  Lane l owns
// the 16-byte group l % 8 of the block and the positions l / 8 + 8 k, k < L
// (positions past P re-read position 0, in bounds, and count as zero); the
// 8 lanes of a group add their sums with xor shuffles (offsets 8, 16, 32,
// a fixed order), and lanes 0..7 write the block's 64 means.  No LDS, no
// barrier; four independent waves per workgroup.  Measured on MI355X,
// back to back ([128, 1536, h, w], the nfnet corpus images; the block
// kernel's time first): 6x6 5.47 -> 4.56 us, 7x7 6.33 -> 5.28, 8x8 6.63 ->
// 5.96, 9x9 8.06 -> 7.16, 12x12 12.36 -> 10.90 (Inductor 4.78, 5.29, 6.48,
// 7.58, 12.17); blocks of 128 or 256 channels (16 or 32 lanes per row)
// were slower (4.85 / 5.50 us at 6x6).  Up to 224 positions (28 loads per
// lane): [128, 1536, 14, 14] 15.3 -> 13.8 us back to back (18.3 -> 16.8
// after a cache flush), [64, 1536, 14, 15] 10.5 -> 9.0.
constexpr int kSmallGroups = 8;    // 16-byte groups per wave block (64 channels)
constexpr int kSmallMaxLoads = 28;  // positions per lane: P <= 224

template <int L>
__global__ __launch_bounds__(256) void spatial_mean_small_waves(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ out, int64_t N, int P, int64_t C,
    int cblocks) {
  constexpr int G = kSmallGroups;
  constexpr int kRows = kWave / G;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const bool ok = w < N * cblocks;
  const int64_t wc = ok ? w : 0;
  const int64_t n = wc / cblocks;
  const int cb = static_cast<int>(wc - n * cblocks);
  const int g = cb * G + (lane % G);
  const int r = lane / G;
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x + n * P * C) + g;
  const int64_t G64 = C / 8;
  u32x4_t v[L];
#pragma unroll
  for (int k = 0; k < L; ++k) {
    const int p = r + k * kRows;
    v[k] = __builtin_nontemporal_load(xv + (p < P ? p : 0) * G64);
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < L; ++k) {
    const bool in = r + k * kRows < P;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc[2 * d] += in ? bf16lo(v[k][d]) : 0.f;
      acc[2 * d + 1] += in ? bf16hi(v[k][d]) : 0.f;
    }
  }
  // Add lanes 8, 16 and 32 apart (the same pairs as xor shuffles, so the same
  // sums): row_ror:8 within each 16-lane row, then gfx950's permlane swaps,
  // which hand every lane its partner's value without an LDS round trip.
  static_assert(G == 8, "the combine adds lanes 8 apart first");
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += dpp<kDppRowRor8>(acc[e]);
    const auto h = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[e]),
                                                    __float_as_uint(acc[e]), false, false);
    acc[e] = __uint_as_float(h[0]) + __uint_as_float(h[1]);
    const auto w = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e]),
                                                    __float_as_uint(acc[e]), false, false);
    acc[e] = __uint_as_float(w[0]) + __uint_as_float(w[1]);
  }
  if (ok && lane < G) {
    const float inv = 1.0f / static_cast<float>(P);
    u32x4_t o;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = pack_bf16x2(acc[2 * d] * inv, acc[2 * d + 1] * inv);
    *reinterpret_cast<u32x4_t*>(out + n * C + 8 * g) = o;
  }
}

// out[n, c] = bf16(sum_s partial[n, s, c] / P), slices added in order.
__global__ __launch_bounds__(256) void spatial_mean_finish(
    const float* __restrict__ partial, uint16_t* __restrict__ out, int64_t N,
    int64_t P, int64_t C, int slices) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * C) return;
  const int64_t n = i / C, c = i - n * C;
  const float* src = partial + n * slices * C + c;
  float sum = src[0];
  for (int s = 1; s < slices; ++s) sum += src[static_cast<int64_t>(s) * C];
  out[i] = static_cast<uint16_t>(pack_bf16x2(sum / static_cast<float>(P), 0.f) & 0xffffu);
}

// Any C: one thread per (n, c), strided loads.
__global__ __launch_bounds__(256) void spatial_mean_nhwc_scalar(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ out, int64_t N,
    int64_t P, int64_t C) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * C) return;
  const int64_t n = i / C, c = i - n * C;
  const uint16_t* src = x + n * P * C + c;
  float sum = 0.f;
  for (int64_t p = 0; p < P; ++p) sum += bf16_to_f32(src[p * C]);
  out[i] = static_cast<uint16_t>(pack_bf16x2(sum / static_cast<float>(P), 0.f) & 0xffffu);
}

int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Threads per workgroup, channel blocks and position slices per image for
// the vector path (0 threads: use the scalar kernel).
struct SpatialPlan {
  int threads = 0;
  int group_block = 0;  // 16-byte channel groups per workgroup
  int cblocks = 1;      // channel blocks per image
  int slices = 1;
  int64_t slice_len = 0;
};

// Channel blocks of 64 groups (1 KiB of each row), or of 32 (512 bytes),
// or of 16 (256 bytes),
// when the row divides into them and images x blocks give at least 256
// workgroups: no position split, so no partial sums and no second kernel.
// 64-group blocks are tried first, except for small images (below).
// The workgroup takes R rows per instruction, the smallest power of two
// that covers the image's positions in four rounds of kUnroll loads per
// thread, at most 512 threads.
// Measured on MI355X (oracle runner, cold cache): 64-group blocks 5-15 %
// faster than two position slices plus the finishing kernel on the eight
// 1536-channel corpus points (e.g. [128, 1536, 8, 8] 11.2 -> 9.6 us,
// [128, 1536, 18, 18] 26.7 -> 24.7 us); R sized to the positions instead
// of a fixed 8 rows, [128, 1536, 6, 6] 15.4 -> 15.1 us and [128, 512, 24,
// 24] (32-group blocks instead of slices) 25.1 -> 23.7 us (graph replays);
// one round (R up to 16 rows, 1024 threads) was 4-6 % slower, cached loads
// and 16- or 8-group blocks no faster where 64-group blocks apply.
constexpr int kChannelBlock = 64;

SpatialPlan spatial_plan(int64_t n, int64_t p, int64_t c) {
  SpatialPlan plan;
  if (c % 8 != 0 || c / 8 > kMaxThreads || n <= 0 || p <= 0) return plan;
  // Small images (at most 128 positions) take 32-group blocks first: twice
  // the workgroups for the same bytes ([128, 1536, 9, 9] 8.53 -> 8.03 us,
  // [128, 1536, 8, 8] 6.81 -> 6.60, [128, 1536, 6, 6] 5.68 -> 5.52 in the
  // steady loop; larger images unchanged).
  // Then 16-group blocks (256 bytes of each row), where the wider blocks
  // give too few workgroups: C = 256 at 128 images takes 256 workgroups
  // with no position slices and no finishing kernel ([128, 256, 72, 72]
  // 57.9 -> 56.1 us after a cache flush, 55.2 -> 53.0 back to back;
  // [128, 256, 56, 56] 37.8 -> 36.4 / 34.7 -> 33.4; [128, 256, 48, 48] and
  // [128, 256, 64, 64] 1-3 % faster).
  const int first = p <= 128 ? kChannelBlock / 2 : kChannelBlock;
  const int gbs[3] = {first, kChannelBlock + kChannelBlock / 2 - first, kChannelBlock / 4};
  for (const int gb : gbs) {
    if ((c / 8) % gb != 0 || n * (c / 8 / gb) < 256) continue;
    int64_t r = 1;
    while (r * kUnroll * 4 < p && gb * r * 2 <= 512) r *= 2;
    while (gb * r % kWave != 0) r *= 2;  // whole waves
    plan.group_block = gb;
    plan.cblocks = static_cast<int>(c / 8 / gb);
    plan.threads = static_cast<int>(gb * r);
    plan.slices = 1;
    plan.slice_len = p;
    return plan;
  }
  const int64_t G = c / 8;
  plan.group_block = static_cast<int>(G);
  const int64_t lcm = G / gcd64(G, kWave) * kWave;
  int64_t T = lcm <= kMaxThreads ? lcm * std::max<int64_t>(1, 512 / lcm) : G;
  const int64_t rows = T / G;
  if (rows > p) T = G * std::max<int64_t>(1, p);  // no more rows than positions
  plan.threads = static_cast<int>(std::min<int64_t>(T, kMaxThreads));
  const int64_t R = plan.threads / G;
  // About 256 workgroups, each slice at least 4 loads per thread deep and
  // the fp32 partials at most ~6 % of the input traffic (2 S / P).
  int64_t S = std::min<int64_t>((256 + n - 1) / n, std::max<int64_t>(1, p / (4 * R)));
  S = std::max<int64_t>(1, std::min<int64_t>(S, p / 32));
  plan.slices = static_cast<int>(S);
  plan.slice_len = (p + S - 1) / S;
  return plan;
}

// The small-image kernel's loads per lane (ceil(P / 8)), or 0 where it
// does not apply: C a multiple of 64, P <= 224, and at least 512 waves (two
// per CU) of (image, 64-channel block).
int spatial_small_loads(int64_t n, int64_t p, int64_t c) {
  if (c % (8 * kSmallGroups) != 0 || p <= 0 || n <= 0) return 0;
  const int64_t rows = kWave / kSmallGroups;
  const int64_t loads = (p + rows - 1) / rows;
  if (loads > kSmallMaxLoads || n * (c / (8 * kSmallGroups)) < 512) return 0;
  return static_cast<int>(loads);
}

void launch_small_waves(int loads, const uint16_t* x, uint16_t* out, int64_t n, int p, int64_t c,
                        hipStream_t stream) {
  const int cblocks = static_cast<int>(c / (8 * kSmallGroups));
  const dim3 grid(static_cast<unsigned>((n * cblocks + 3) / 4));
#define HIPO_SMW(L_) \
  spatial_mean_small_waves<L_><<<grid, dim3(256), 0, stream>>>(x, out, n, p, c, cblocks)
  switch (loads) {
    case 1: HIPO_SMW(1); break;
    case 2: HIPO_SMW(2); break;
    case 3: HIPO_SMW(3); break;
    case 4: HIPO_SMW(4); break;
    case 5: HIPO_SMW(5); break;
    case 6: HIPO_SMW(6); break;
    case 7: HIPO_SMW(7); break;
    case 8: HIPO_SMW(8); break;
    case 9: case 10: HIPO_SMW(10); break;
    case 11: case 12: HIPO_SMW(12); break;
    case 13: case 14: HIPO_SMW(14); break;
    case 15: case 16: HIPO_SMW(16); break;
    case 17: case 18: HIPO_SMW(18); break;
    case 19: case 20: HIPO_SMW(20); break;
    case 21: case 22: case 23: case 24: HIPO_SMW(24); break;
    default: HIPO_SMW(28); break;
  }
#undef HIPO_SMW
}

}  // namespace
}  // namespace hipo

extern "C" size_t hipo_spatial_mean_workspace_bytes(int64_t n, int64_t hw, int64_t c) {
  if (hipo::spatial_small_loads(n, hw, c) > 0) return 0;
  const hipo::SpatialPlan plan = hipo::spatial_plan(n, hw, c);
  if (plan.threads == 0 || plan.slices <= 1) return 0;
  return static_cast<size_t>(n * plan.slices * c) * sizeof(float);
}

extern "C" int hipo_spatial_mean_nhwc_bf16(const uint16_t* x, uint16_t* out, int64_t n,
                                          int64_t hw, int64_t c, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n >= 0 && hw >= 0 && c >= 0, "spatial_mean: negative size");
  if (n == 0 || c == 0) return 0;
  HIPO_REQUIRE(hw > 0, "spatial_mean: empty spatial extent");
  HIPO_REQUIRE(x && out, "spatial_mean: null pointer");
  if (const int loads = spatial_small_loads(n, hw, c); loads > 0 && aligned16(x) && aligned16(out)) {
    HIPO_REQUIRE((n * (c / 64) + 3) / 4 <= 0x7fffffff, "spatial_mean: too many images");
    launch_small_waves(loads, x, out, n, static_cast<int>(hw), c, stream);
    return check_launch("spatial_mean_nhwc_bf16");
  }
  const SpatialPlan plan = spatial_plan(n, hw, c);
  if (plan.threads > 0 && aligned16(x) && aligned16(out)) {
    const size_t need = plan.slices > 1 ? static_cast<size_t>(n * plan.slices * c) * 4 : 0;
    HIPO_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                 "spatial_mean: workspace of %zu bytes, need %zu", workspace_bytes, need);
    const int64_t blocks = n * plan.cblocks * plan.slices;
    HIPO_REQUIRE(blocks <= 0x7fffffff, "spatial_mean: too many images");
    const int G = plan.group_block;
    const int R = plan.threads / G;
    const size_t lds = R > 1 ? static_cast<size_t>(plan.threads) * 8 * sizeof(float) : 0;
    spatial_mean_nhwc_partial<<<dim3(static_cast<unsigned>(blocks)), dim3(plan.threads), lds,
                                stream>>>(x, out, static_cast<float*>(workspace), hw, c, G,
                                          plan.cblocks, plan.slices, plan.slice_len);
    if (plan.slices > 1) {
      const int64_t total = n * c;
      spatial_mean_finish<<<dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                            stream>>>(static_cast<const float*>(workspace), out, n, hw, c,
                                      plan.slices);
    }
  } else {
    const int64_t total = n * c;
    HIPO_REQUIRE((total + 255) / 256 <= 0x7fffffff, "spatial_mean: too large");
    spatial_mean_nhwc_scalar<<<dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                               stream>>>(x, out, n, hw, c);
  }
  return check_launch("spatial_mean_nhwc_bf16");
}
