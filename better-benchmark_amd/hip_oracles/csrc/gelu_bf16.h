// bf16 -> bf16 GELU(tanh) by bit pattern: the correctly rounded result of
// GELU_tanh(t) = 0.5 t (1 + tanh(sqrt(2/pi) (t + 0.044715 t^3))) for every
// bf16 input t, with no transcendental evaluated on the device.
//   2^-10 <= |t| < 16 (3584 inputs): read from a table of the correctly
//     rounded results (gelu_table.h, generated at 96-bit precision), which
//     the kernels stage in LDS;
//   2^-125 <= |t| < 2^-10: t / 2, an exponent decrement (GELU(t) = t/2 (1 +
//     u + ...) with |u| < 0.8 * 2^-10, less than half a bf16 ulp, and t / 2
//     is a bf16 value);
//   t >= 16: t (1 - GELU(t) / t < e^-300);  t <= -16: -0 (|GELU(t)| <
//     e^-300 underflows);  +inf -> +inf, -inf -> NaN (as -inf * 0 in
//     eager), NaN -> NaN;
//   |t| < 2^-125 (bf16 subnormal t / 2): t / 2 rounded to nearest even.
// gen_gelu_table.py --check verifies the whole mapping against the exact
// function.  Eager and Inductor evaluate the tanh form in fp32 and differ
// from it by one ulp within a few fp32 ulps of a rounding boundary and in
// the far negative tail, where their 1 + tanh(u) cancels.
#pragma once

#include "gelu_table.h"
#include "hipo_common.h"

namespace hipo {

constexpr uint32_t kGeluLo = static_cast<uint32_t>(kGeluTableExpLo) << 7;  // |t| = 2^-10

// The table's 16-byte chunks, for staging it into LDS.
constexpr int kGeluTableChunks = kGeluTableSize * 2 / 16;

// The table's inputs (2^-10 <= |t| < 16): a pure lookup.  Branch-free: the
// LDS index is clamped into the table (inputs outside it read an arbitrary
// entry, which gelu_rare() flags for replacement).  `lut` holds kGeluTable.
__device__ __forceinline__ uint32_t gelu_lookup(uint32_t tb, const uint16_t* lut) {
  const uint32_t off = (tb & 0x7fffu) - kGeluLo;  // wraps below the table
  const uint32_t idx = __builtin_elementwise_min(off, static_cast<uint32_t>(kGeluTablePerSign - 1)) +
                       (tb >> 15) * static_cast<uint32_t>(kGeluTablePerSign);
  return lut[idx];
}

// Inputs outside the table: |t| < 2^-10 (zero included), |t| >= 16, inf,
// NaN -- the same offset test as the lookup's clamp.
__device__ __forceinline__ bool gelu_rare(uint32_t tb) {
  return ((tb & 0x7fffu) - kGeluLo) >= static_cast<uint32_t>(kGeluTablePerSign);
}

__device__ __forceinline__ uint32_t gelu_bits_rare(uint32_t tb) {
  const uint32_t mag = tb & 0x7fffu;
  if (mag < 0x100u)  // +-0 and subnormal results: t / 2 rounded to nearest even
    return pack_bf16x2(0.5f * bf16_to_f32(static_cast<uint16_t>(tb)), 0.0f) & 0xffffu;
  if (mag < kGeluLo) return tb - 0x80u;                  // t / 2, an exponent decrement
  if ((tb & 0x8000u) == 0 || mag > 0x7f80u) return tb;  // t >= 16, +inf, NaN
  return mag == 0x7f80u ? 0x7fc0u : 0x8000u;             // -inf -> NaN; t <= -16 -> -0
}

__device__ __forceinline__ uint32_t gelu_bits(uint32_t tb, const uint16_t* lut) {
  return gelu_rare(tb) ? gelu_bits_rare(tb) : gelu_lookup(tb, lut);
}

// Both halves of a word of two bf16 values.
__device__ __forceinline__ uint32_t gelu_pair_common(uint32_t w, const uint16_t* lut) {
  return gelu_lookup(w & 0xffffu, lut) | (gelu_lookup(w >> 16, lut) << 16);
}
__device__ __forceinline__ bool gelu_pair_rare(uint32_t w) {
  return gelu_rare(w & 0xffffu) | gelu_rare(w >> 16);
}
__device__ __forceinline__ uint32_t gelu_pair(uint32_t w, const uint16_t* lut) {
  return gelu_bits(w & 0xffffu, lut) | (gelu_bits(w >> 16, lut) << 16);
}

}  // namespace hipo
