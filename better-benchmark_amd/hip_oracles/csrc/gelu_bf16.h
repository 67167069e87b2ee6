// bf16 -> bf16 GELU(tanh) by bit pattern: the correctly rounded result of
// GELU_tanh(t) = 0.5 t (1 + tanh(sqrt(2/pi) (t + 0.044715 t^3))) for every
// bf16 input t.
//
// Common inputs (t > -4, the bulk of any activation): an fp32 evaluation
// without a table, gelu_tanh_fast() below, rounded once to bf16.  Its
// result is the correctly rounded one for every bf16 t > -4: the tests run
// all 65,536 bf16 inputs through every kernel that uses it and compare bit
// for bit with the correctly rounded table (the GPU's exp2 / rcp are
// deterministic, and the bf16 domain is finite, so that comparison is the
// proof).  On the CPU, with exp2 and rcp rounded correctly, the closest any
// of these results comes to a bf16 rounding boundary is 12 fp32 ulps, while
// the evaluation's error there is a few ulps.
//
// Rare inputs (t <= -4, -inf, NaN): the exact map, gelu_bits() (gelu_exact_x8()
// for 8 values at once):
//   2^-10 <= |t| < 16 (3584 inputs): read from a table of the correctly
//     rounded results (gelu_table.h, generated at 96-bit precision) in
//     global memory (7 KiB, cache-resident);
//   2^-125 <= |t| < 2^-10: t / 2, an exponent decrement (GELU(t) = t/2 (1 +
//     u + ...) with |u| < 0.8 * 2^-10, less than half a bf16 ulp, and t / 2
//     is a bf16 value);
//   t >= 16: t (1 - GELU(t) / t < e^-300);  t <= -16: -0 (|GELU(t)| <
//     e^-300 underflows);  +inf -> +inf, -inf -> NaN (as -inf * 0 in
//     eager), NaN -> NaN;
//   |t| < 2^-125 (bf16 subnormal t / 2): t / 2 rounded to nearest even.
// Below -4 the fp32 form's exponent argument grows (|z| > 16; exp2 then
// amplifies its rounding error) and past t = -10 exp2 overflows while the
// exact result is still a normal or subnormal bf16, so those inputs take the
// exact map.  gen_gelu_table.py --check verifies the whole exact mapping
// against the exact function.  Eager and Inductor evaluate the tanh form in
// fp32 and differ from it by one ulp within a few fp32 ulps of a rounding
// boundary and in the far negative tail, where their 1 + tanh(u) cancels.
#pragma once

#include "gelu_table.h"
#include "hipo_common.h"

namespace hipo {

constexpr uint32_t kGeluLo = static_cast<uint32_t>(kGeluTableExpLo) << 7;  // |t| = 2^-10

// The table's inputs (2^-10 <= |t| < 16): a pure lookup.  Branch-free: the
// index is clamped into the table (inputs outside it read an arbitrary
// entry, which gelu_rare() flags for replacement).  `lut` is kGeluTable.
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

// gelu_tanh_fast(t) = t / (1 + e^(-2u)) = t / (1 + 2^z), z = t (K0 + K1 t^2),
// K0 = -2 sqrt(2/pi) / ln 2, K1 = 0.044715 K0 (0.5 t (1 + tanh u) = t
// sigmoid(2u), exactly; this form does not cancel for negative t): the
// hardware exp2 (v_exp_f32) and reciprocal (v_rcp_f32).  t^2 is exact for a
// bf16 t.  Used only for t > kGeluFastMin, where it gives the correctly
// rounded bf16 result (see the top of this file).
constexpr float kGeluK0 = -2.3022081981443248f;
constexpr float kGeluK1 = -0.1029432395800235f;
constexpr float kGeluFastMin = -4.0f;

__device__ __forceinline__ float gelu_tanh_fast(float t) {
  const float z = t * __builtin_fmaf(kGeluK1, t * t, kGeluK0);
  return t * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

// Both halves of a word of two bf16 t: the fast form, packed; `rare` is set
// when either t needs the exact map (t <= -4, -inf, NaN: the comparison is
// false for NaN).
__device__ __forceinline__ uint32_t gelu_pair_fast(uint32_t w, bool& rare) {
  const float t0 = bf16lo(w);
  const float t1 = bf16hi(w);
  rare |= !(t0 > kGeluFastMin) | !(t1 > kGeluFastMin);
  return pack_bf16x2(gelu_tanh_fast(t0), gelu_tanh_fast(t1));
}

// The exact map of the 8 values in 4 words, from the table in global memory
// (the rare path of the fast kernels): the 8 clamped table reads (always in
// bounds) are issued together, then each result is selected -- one wait for
// the loads instead of one per value.
__device__ __forceinline__ void gelu_exact_x8(const u32x4_t& w, u32x4_t& o) {
  uint32_t tab[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    tab[2 * k] = gelu_lookup(w[k] & 0xffffu, kGeluTable);
    tab[2 * k + 1] = gelu_lookup(w[k] >> 16, kGeluTable);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = w[k] & 0xffffu;
    const uint32_t hi = w[k] >> 16;
    const uint32_t rlo = gelu_rare(lo) ? gelu_bits_rare(lo) : tab[2 * k];
    const uint32_t rhi = gelu_rare(hi) ? gelu_bits_rare(hi) : tab[2 * k + 1];
    o[k] = rlo | (rhi << 16);
  }
}

}  // namespace hipo
