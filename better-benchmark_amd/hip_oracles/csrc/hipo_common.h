// Shared device helpers and host-side error plumbing for libhip_oracles.
//
// Written for gfx950 (CDNA4): wave64, 16-byte global loads/stores, DPP
// cross-lane reductions, hardware bf16 conversion (v_cvt_pk_bf16_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "hip_oracles.h"

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local message; see hipo_last_error()).
// ---------------------------------------------------------------------------
namespace hipo {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Properties of the current device, cached per device on first use.
struct DeviceInfo {
  int device;
  int cu_count;          // multiProcessorCount
  int max_threads_per_cu;
  size_t lds_per_block;  // sharedMemPerBlock
};
const DeviceInfo* device_info();

// Map the result of a kernel launch onto the ABI's return convention.
int check_launch(const char* what);

}  // namespace hipo

#define HIPO_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::hipo::set_error(__VA_ARGS__);    \
      return HIPO_EINVAL;                \
    }                                    \
  } while (0)

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
namespace hipo {

constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
// 16-byte vectors as native clang vectors (the non-temporal load/store
// builtins accept these, not HIP's struct vector types).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

inline bool aligned16(const void* p) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0;
}
inline bool aligned8(const void* p) {
  return reinterpret_cast<uintptr_t>(p) % 8 == 0;
}

// bf16 bits held in the low / high half of a 32-bit word -> fp32 (exact).
__device__ __forceinline__ float bf16lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Two fp32 -> one word of two bf16 (round to nearest even, NaN stays NaN):
// a single v_cvt_pk_bf16_f32 on gfx950.  `lo` lands in bits 0..15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  float2_t v = {lo, hi};
  bf16x2_t b = __builtin_convertvector(v, bf16x2_t);
  return __builtin_bit_cast(uint32_t, b);
}

// fp32 -> fp32 value rounded through bf16 (what an eager bf16 op stores).
__device__ __forceinline__ float round_bf16(float v) {
  return bf16lo(pack_bf16x2(v, 0.0f));
}

// Division of numerators n < 2^31 by a runtime divisor d >= 1 as
// (n * magic) >> shift, shift = 31 + ceil(log2 d), magic = ceil(2^shift / d):
// exact, since magic * d - 2^shift = e <= d and n * e < 2^shift.  The
// hardware has no integer divide; this replaces a ~30-instruction sequence
// with one 64-bit multiply where a kernel divides before its first load.
struct DivMagic {
  uint32_t magic;
  int shift;
};

inline DivMagic div_magic(uint32_t d) {
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  const int shift = 31 + l;
  return DivMagic{static_cast<uint32_t>(((uint64_t{1} << shift) + d - 1) / d), shift};
}

__device__ __forceinline__ uint32_t div_by(uint32_t n, DivMagic m) {
  return static_cast<uint32_t>((static_cast<uint64_t>(n) * m.magic) >> m.shift);
}

// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;  // row_ror:4
constexpr int kDppRowRor8 = 0x128;  // row_ror:8

constexpr int kDppRowHalfMirror = 0x141;  // row_half_mirror: lane i of 8 <- lane 7 - i

template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

template <int Ctrl>
__device__ __forceinline__ double dpp(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b)), Ctrl, 0xF, 0xF,
                                  false));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b >> 32)), Ctrl,
                                  0xF, 0xF, false));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Sum over each aligned group of 8 lanes, every lane of the group receiving
// it (quad butterflies, then the mirrored half-row); all 64 lanes active.
// Every lane adds the same two values at each step (a + b = b + a), so the
// 8 results are identical.
template <typename T>
__device__ __forceinline__ T sum8(T v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowHalfMirror>(v);
  return v;
}

// Full-wave sum; every lane receives the same value.  All 64 lanes must be
// active.  Order is fixed (DPP butterflies within each 16-lane row, then
// (row0 + row1) + (row2 + row3)), so results are deterministic.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowRor4>(v);
  v += dpp<kDppRowRor8>(v);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

// The same fixed-order full-wave sum in fp64.
__device__ __forceinline__ double wave_sum(double v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowRor4>(v);
  v += dpp<kDppRowRor8>(v);
  auto lane_value = [&](int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), l));
    const uint32_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), l));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
  };
  return (lane_value(0) + lane_value(16)) + (lane_value(32) + lane_value(48));
}

// Full-wave max; every lane receives the same value (all lanes active).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppRowRor4>(v));
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Full-wave maximum with NaN propagation (IEEE 754-2019 maximum: NaN if
// any lane holds NaN; v_maximum3_f32 on gfx950, so no operand
// canonicalisation as fmaxf needs); every lane receives it.
__device__ __forceinline__ float wave_maximum(float v) {
  v = __builtin_elementwise_maximum(v, dpp<kDppQuadXor1>(v));
  v = __builtin_elementwise_maximum(v, dpp<kDppQuadXor2>(v));
  v = __builtin_elementwise_maximum(v, dpp<kDppRowRor4>(v));
  v = __builtin_elementwise_maximum(v, dpp<kDppRowRor8>(v));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b),
                                       __builtin_elementwise_maximum(c, d));
}

// e^x in fp32 to about one ulp, for x in [-104, 89] (NaN propagates), by
// a Cody-Waite reduction: ph = x * log2(e) rounded (any rounding of it is
// absorbed below), r = x - ph * ln2 with ln2 split into hi + lo (two FMAs;
// the first is exact to within 2^-24 of its tiny result, so r carries
// x's full precision: |r| <= ~6e-6 here, accurate to ~1e-13), and
// e^x = 2^ph * e^r with 2^ph from the hardware exp2 and e^r = 1 + r
// (r^2 / 2 <= 2e-11 is below fp32's 2^-24).  exp_f32 forms 2^ph * (1 + r):
// the product keeps 2^ph = inf (x up to 89: e^89 overflows) and 2^ph = 0
// exact; exp_f32_nonpos, for x <= 0 only (2^ph <= 1, never inf), forms
// fma(2^ph, r, 2^ph), one instruction and one rounding fewer (the fma
// would give inf * r + inf = NaN for an overflowed 2^ph and r <= 0).
// Results below 2^-126 (x < -87.3) are whatever the hardware exp2 gives
// there (denormal or zero) -- below any bf16 rounding these kernels apply.
// Callers clamp x first (exp_domain, or at -104 for exp_f32_nonpos):
// e^-104 rounds to 0, e^89 overflows to inf.
constexpr float kLog2eHi = 1.4426950216293335f;   // log2(e) rounded to fp32
constexpr float kLn2Hi = 0.6931471824645996f;     // ln 2 rounded to fp32
constexpr float kLn2Lo = -1.9046542121259336e-09f;  // ln 2 - kLn2Hi, rounded
__device__ __forceinline__ float exp_reduce(float x, float& ph) {
  ph = x * kLog2eHi;
  return __builtin_fmaf(-ph, kLn2Lo, __builtin_fmaf(-ph, kLn2Hi, x));
}
__device__ __forceinline__ float exp_f32(float x) {
  float ph;
  const float r = exp_reduce(x, ph);
  return __builtin_amdgcn_exp2f(ph) * (1.0f + r);
}
__device__ __forceinline__ float exp_f32_nonpos(float x) {
  float ph;
  const float r = exp_reduce(x, ph);
  const float e = __builtin_amdgcn_exp2f(ph);
  return __builtin_fmaf(e, r, e);
}

// e / sum correctly rounded (the IEEE quotient), given inv = 1 / sum
// correctly rounded: q = e * inv is within 1.5 ulp of e / sum, and one FMA
// step with the exact remainder e - q * sum gives the rounded quotient
// (Markstein's correction; pinned against exact rational arithmetic over
// the softmax domain, e in (0, 1], sum in [1, 2048], by a CPU test).  2
// FMAs per element where a full division takes ~10 instructions.
__device__ __forceinline__ float div_rn(float e, float sum, float inv) {
  const float q = e * inv;
  return __builtin_fmaf(__builtin_fmaf(-q, sum, e), inv, q);
}

// Clamp to the domain of exp_f32; NaN stays NaN (IEEE 754-2019 maximum /
// minimum: v_maximum3_f32 / v_minimum3_f32 on gfx950).
__device__ __forceinline__ float exp_domain(float x) {
  return __builtin_elementwise_minimum(__builtin_elementwise_maximum(x, -104.0f), 89.0f);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace hipo
