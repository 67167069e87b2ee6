// GELU(tanh) of a contiguous tensor, element by element (no layout change).
//
// bf16: y = the correctly rounded bf16 GELU_tanh(x) for every bf16 x, by bit
//   pattern (gelu_bf16.h): an fp32 evaluation that rounds correctly for
//   x > -4, the exact table in global memory below that.  The
//   repro's eager graph rounds every intermediate to bf16 (its 1 + tanh(u)
//   cancels in the negative tail); Inductor and the reference's Triton
//   oracle evaluate the chain in fp32 and round once -- the exact result is
//   what both approximate.
// fp32: the same function in its non-cancelling form,
//     y = x / (1 + e^(-2u)),  u = 0.7978845608028654 (x + 0.044715 x^3)
//   (0.5 x (1 + tanh u) = x sigmoid(2u), exactly), with the
//   extended-precision exp_f32 and an IEEE division: a few fp32 ulps from
//   the exact value everywhere, where eager's and Inductor's 1 + tanh(u)
//   cancels in the negative tail.  The device library's tanhf (what they
//   call) costs about twice the instructions, and without packed FP32 math
//   that made this kernel VALU-bound (65.8 us at the FNet point against
//   Inductor's 67.6 us graph replay, whose kernel uses packed fp32 ops).
//
// Layout: each wave64 moves a contiguous run of U KiB (U 1 KiB sub-chunks,
// lane l taking the 16-byte vector l of each), loads issued together, four
// waves per 256-thread workgroup, a one-shot grid in memory order; loads are
// non-temporal, and so are the bf16 kernel's stores.  The fp32 kernel's
// stores are cached: at the FNet point [16384, 3072] they take the
// reference harness's clean-cache launch from 73.7 to 69.0 us (graph
// replay; Inductor 67.6), at a cost in the back-to-back loop (67.0 -> 70.0
// us), where non-temporal stores win.  Elements past the last whole 16-byte vector are
// done one by one by a second, one-workgroup launch.
// HBM-bound: algorithmic bytes per element = 2 x sizeof(element).
#include "gelu_bf16.h"
#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kGeluWaves = 4;
constexpr int kGeluThreads = kGeluWaves * kWave;

template <int U>
__global__ __launch_bounds__(kGeluThreads) void gelu_bf16_flat(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int64_t nvec) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t v0 =
      (static_cast<int64_t>(blockIdx.x) * kGeluWaves + (threadIdx.x >> 6)) * (U * kWave) + lane;
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x);
  u32x4_t* yv = reinterpret_cast<u32x4_t*>(y);

  u32x4_t v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // Slots past the end load the last vector (in bounds) and store nothing.
    const int64_t i = v0 + u * kWave;
    v[u] = __builtin_nontemporal_load(xv + (i < nvec ? i : nvec - 1));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = v0 + u * kWave;
    u32x4_t o;
    bool rare = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = gelu_pair_fast(v[u][k], rare);
    if (rare) {  // one branch per 8 values, rarely taken for ordinary data
      gelu_exact_x8(v[u], o);
    }
    if (i < nvec) __builtin_nontemporal_store(o, yv + i);
  }
}

// Elements [first, first + count), count < 8, from the table in global memory.
__global__ __launch_bounds__(kWave) void gelu_bf16_tail(const uint16_t* __restrict__ x,
                                                        uint16_t* __restrict__ y,
                                                        int64_t first, int count) {
  if (static_cast<int>(threadIdx.x) < count) {
    const int64_t e = first + threadIdx.x;
    y[e] = static_cast<uint16_t>(gelu_bits(x[e], kGeluTable));
  }
}

// x / (1 + e^(-2u)); e^-2u saturates to 0 (x -> +inf: y = x) and to inf
// (x -> -inf: y = -0, and -inf / inf = NaN as eager's -inf * 0); NaN stays NaN.
__device__ __forceinline__ float gelu_tanh_f32(float x) {
  const float m2u = -1.5957691216057308f * __builtin_fmaf(0.044715f * x, x * x, x);
  return x / (1.0f + exp_f32(exp_domain(m2u)));
}

template <int U>
__global__ __launch_bounds__(kGeluThreads) void gelu_f32_flat(
    const float* __restrict__ x, float* __restrict__ y, int64_t nvec) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t v0 =
      (static_cast<int64_t>(blockIdx.x) * kGeluWaves + (threadIdx.x >> 6)) * (U * kWave) + lane;
  const f32x4_t* xv = reinterpret_cast<const f32x4_t*>(x);
  f32x4_t* yv = reinterpret_cast<f32x4_t*>(y);
  f32x4_t v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = v0 + u * kWave;
    v[u] = __builtin_nontemporal_load(xv + (i < nvec ? i : nvec - 1));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = v0 + u * kWave;
    f32x4_t o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = gelu_tanh_f32(v[u][k]);
    if (i < nvec) yv[i] = o;  // cached stores (see the header comment)
  }
}

__global__ __launch_bounds__(kWave) void gelu_f32_tail(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t first,
                                                       int count) {
  if (static_cast<int>(threadIdx.x) < count) {
    const int64_t e = first + threadIdx.x;
    y[e] = gelu_tanh_f32(x[e]);
  }
}

// Vectors per lane: U KiB per wave, fewer when the tensor would not give
// every CU a few workgroups.
inline int vectors_per_lane(int64_t nvec, int big) {
  const int64_t per_block_big = int64_t{big} * kGeluThreads;
  return (nvec + per_block_big - 1) / per_block_big >= 1024 ? big : 2;
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_gelu_tanh_bf16(const uint16_t* x, uint16_t* y, int64_t n,
                                   hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n >= 0, "gelu_tanh: negative size");
  if (n == 0) return 0;
  HIPO_REQUIRE(x && y, "gelu_tanh: null pointer");
  HIPO_REQUIRE(aligned16(x) && aligned16(y), "gelu_tanh: pointers must be 16-byte aligned");
  const int64_t nvec = n / 8;
  const int tail = static_cast<int>(n % 8);
  if (nvec > 0) {
    const int u = vectors_per_lane(nvec, 8);
    const int64_t per_block = int64_t{u} * kGeluThreads;
    const int64_t blocks = (nvec + per_block - 1) / per_block;
    HIPO_REQUIRE(blocks < (int64_t{1} << 31), "gelu_tanh: too large");
    const dim3 grid(static_cast<unsigned>(blocks)), block(kGeluThreads);
    if (u == 8) {
      gelu_bf16_flat<8><<<grid, block, 0, stream>>>(x, y, nvec);
    } else {
      gelu_bf16_flat<2><<<grid, block, 0, stream>>>(x, y, nvec);
    }
  }
  if (tail > 0) gelu_bf16_tail<<<dim3(1), dim3(kWave), 0, stream>>>(x, y, nvec * 8, tail);
  return check_launch("gelu_tanh_bf16");
}

extern "C" int hipo_gelu_tanh_f32(const float* x, float* y, int64_t n, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n >= 0, "gelu_tanh: negative size");
  if (n == 0) return 0;
  HIPO_REQUIRE(x && y, "gelu_tanh: null pointer");
  HIPO_REQUIRE(aligned16(x) && aligned16(y), "gelu_tanh: pointers must be 16-byte aligned");
  const int64_t nvec = n / 4;
  const int tail = static_cast<int>(n % 4);
  if (nvec > 0) {
    const int u = vectors_per_lane(nvec, 4);
    const int64_t per_block = int64_t{u} * kGeluThreads;
    const int64_t blocks = (nvec + per_block - 1) / per_block;
    HIPO_REQUIRE(blocks < (int64_t{1} << 31), "gelu_tanh: too large");
    const dim3 grid(static_cast<unsigned>(blocks)), block(kGeluThreads);
    if (u == 4) {
      gelu_f32_flat<4><<<grid, block, 0, stream>>>(x, y, nvec);
    } else {
      gelu_f32_flat<2><<<grid, block, 0, stream>>>(x, y, nvec);
    }
  }
  if (tail > 0) gelu_f32_tail<<<dim3(1), dim3(kWave), 0, stream>>>(x, y, nvec * 4, tail);
  return check_launch("gelu_tanh_f32");
}
