// Storage-order dtype casts, bf16 <-> fp32, over n elements of a dense
// tensor (contiguous, channels-last or any other dense non-overlapping
// layout: element i of the input's storage becomes element i of the
// output's, which the caller allocates with the same strides):
//   bf16 -> fp32: exact (the bf16 bits become the high half of the fp32);
//   fp32 -> bf16: round to nearest, ties to even (v_cvt_pk_bf16_f32; NaN
//                 stays NaN).
// The reference's pointwise_04d85912d998 / pointwise_ccd411f2a45d graphs
// (an isolated convert_element_type over weights and activations), and the
// materialisation of pointwise_8bb40810003c.
//
// Layout: a one-shot grid in storage order over quads of 4 elements; lane
// l of a step converts quad (step * 256 + thread), so every load and store
// instruction of a wave is one contiguous run (512 bytes of bf16, 1 KiB of
// fp32), non-temporal; a thread's loads are issued before its stores.
// bf16 -> fp32 one quad per thread, fp32 -> bf16 two: measured on MI355X
// against 1, 2, 4 and 8 quads per thread and ordinary loads and stores
// (the runner's single-launch timing credits ordinary stores, whose lines
// drain from the caches after the timed window -- 120.3 against 121.9 us at
// 131 M elements -- while back-to-back streaming favours non-temporal ones,
// as for every kernel here).  The first layout, 8-element groups written as
// two 16-byte fp32 stores per lane, left every store instruction half-used
// (383.6 against 241.6 us at 262 M).  When both pointers are 16-byte aligned
// the whole quads take that path and the n % 4 tail goes element by element;
// otherwise every element does.  Bytes: 6 per element (HBM-bound).
#include "hipo_common.h"

namespace hipo {
namespace {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kCastThreads = 256;

template <int kSteps>
__device__ __forceinline__ int64_t quad_index(int k) {
  return (static_cast<int64_t>(blockIdx.x) * kSteps + k) * kCastThreads + threadIdx.x;
}

template <bool kNt, typename T>
__device__ __forceinline__ T load_as(const T* p) {
  if constexpr (kNt) return __builtin_nontemporal_load(p);
  else return *p;
}

template <bool kNt, typename T>
__device__ __forceinline__ void store_as(T v, T* p) {
  if constexpr (kNt) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <int kSteps, bool kNtLoad, bool kNtStore>
__global__ __launch_bounds__(kCastThreads) void cast_bf16_f32_vec(
    const u32x2_t* __restrict__ x, f32x4_t* __restrict__ y, int64_t quads) {
  u32x2_t v[kSteps];
#pragma unroll
  for (int k = 0; k < kSteps; ++k) {
    const int64_t q = quad_index<kSteps>(k);
    v[k] = load_as<kNtLoad>(x + (q < quads ? q : quads - 1));
  }
#pragma unroll
  for (int k = 0; k < kSteps; ++k) {
    const int64_t q = quad_index<kSteps>(k);
    if (q < quads)
      store_as<kNtStore>(
          f32x4_t{bf16lo(v[k][0]), bf16hi(v[k][0]), bf16lo(v[k][1]), bf16hi(v[k][1])}, y + q);
  }
}

template <int kSteps, bool kNtLoad, bool kNtStore>
__global__ __launch_bounds__(kCastThreads) void cast_f32_bf16_vec(
    const f32x4_t* __restrict__ x, u32x2_t* __restrict__ y, int64_t quads) {
  f32x4_t v[kSteps];
#pragma unroll
  for (int k = 0; k < kSteps; ++k) {
    const int64_t q = quad_index<kSteps>(k);
    v[k] = load_as<kNtLoad>(x + (q < quads ? q : quads - 1));
  }
#pragma unroll
  for (int k = 0; k < kSteps; ++k) {
    const int64_t q = quad_index<kSteps>(k);
    if (q < quads)
      store_as<kNtStore>(
          u32x2_t{pack_bf16x2(v[k][0], v[k][1]), pack_bf16x2(v[k][2], v[k][3])}, y + q);
  }
}

constexpr int kB2FSteps = 1;
constexpr int kF2BSteps = 2;

// Elements [first, n), one per thread.
__global__ __launch_bounds__(kCastThreads) void cast_bf16_f32_scalar(
    const uint16_t* __restrict__ x, float* __restrict__ y, int64_t first, int64_t n) {
  const int64_t i = first + static_cast<int64_t>(blockIdx.x) * kCastThreads + threadIdx.x;
  if (i < n) y[i] = bf16_to_f32(x[i]);
}

__global__ __launch_bounds__(kCastThreads) void cast_f32_bf16_scalar(
    const float* __restrict__ x, uint16_t* __restrict__ y, int64_t first, int64_t n) {
  const int64_t i = first + static_cast<int64_t>(blockIdx.x) * kCastThreads + threadIdx.x;
  if (i < n) y[i] = static_cast<uint16_t>(pack_bf16x2(x[i], 0.0f) & 0xffffu);
}

unsigned blocks_for(int64_t items, int64_t per_block) {
  return static_cast<unsigned>((items + per_block - 1) / per_block);
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_cast_bf16_to_f32(const uint16_t* x, float* y, int64_t n,
                                     hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n >= 0, "cast_bf16_to_f32: negative size");
  if (n == 0) return 0;
  HIPO_REQUIRE(x && y, "cast_bf16_to_f32: null pointer");
  HIPO_REQUIRE(n / (4 * kCastThreads) < 0x7fffffff, "cast_bf16_to_f32: too many elements");
  int64_t done = 0;
  if (aligned16(x) && aligned16(y)) {
    const int64_t quads = n / 4;
    if (quads > 0)
      cast_bf16_f32_vec<kB2FSteps, true, true>
          <<<blocks_for(quads, static_cast<int64_t>(kCastThreads) * kB2FSteps), kCastThreads, 0,
             stream>>>(reinterpret_cast<const u32x2_t*>(x), reinterpret_cast<f32x4_t*>(y), quads);
    done = quads * 4;
  }
  if (done < n)
    cast_bf16_f32_scalar<<<blocks_for(n - done, kCastThreads), kCastThreads, 0, stream>>>(
        x, y, done, n);
  return check_launch("cast_bf16_to_f32");
}

extern "C" int hipo_cast_f32_to_bf16(const float* x, uint16_t* y, int64_t n,
                                     hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n >= 0, "cast_f32_to_bf16: negative size");
  if (n == 0) return 0;
  HIPO_REQUIRE(x && y, "cast_f32_to_bf16: null pointer");
  HIPO_REQUIRE(n / (4 * kCastThreads) < 0x7fffffff, "cast_f32_to_bf16: too many elements");
  int64_t done = 0;
  if (aligned16(x) && aligned16(y)) {
    const int64_t quads = n / 4;
    if (quads > 0)
      cast_f32_bf16_vec<kF2BSteps, true, true>
          <<<blocks_for(quads, static_cast<int64_t>(kCastThreads) * kF2BSteps), kCastThreads, 0,
             stream>>>(reinterpret_cast<const f32x4_t*>(x), reinterpret_cast<u32x2_t*>(y), quads);
    done = quads * 4;
  }
  if (done < n)
    cast_f32_bf16_scalar<<<blocks_for(n - done, kCastThreads), kCastThreads, 0, stream>>>(
        x, y, done, n);
  return check_launch("cast_f32_to_bf16");
}
