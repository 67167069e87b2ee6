// Welford triples (count, mean, M2) for the BatchNorm statistics: Chan et
// al.'s pairwise merge and a fixed-order wave64 reduction.
#pragma once

#include "hipo_common.h"

namespace hipo {

struct Welford {
  float n;
  float mean;
  float m2;
};

// Chan et al. pairwise merge of two triples over disjoint sets.
__device__ __forceinline__ Welford welford_merge(Welford a, Welford b) {
  const float n = a.n + b.n;
  if (n == 0.f) return a;
  const float wb = b.n / n;
  const float d = b.mean - a.mean;
  Welford r;
  r.n = n;
  r.mean = __builtin_fmaf(d, wb, a.mean);
  r.m2 = a.m2 + b.m2 + d * d * a.n * wb;
  return r;
}

template <int Ctrl>
__device__ __forceinline__ Welford welford_dpp(Welford w) {
  return Welford{dpp<Ctrl>(w.n), dpp<Ctrl>(w.mean), dpp<Ctrl>(w.m2)};
}

__device__ __forceinline__ Welford welford_lane(Welford w, int lane) {
  return Welford{
      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w.n), lane)),
      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w.mean), lane)),
      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w.m2), lane))};
}

// Whole-wave merge (all 64 lanes active); every lane gets the result.  Each
// step merges triples over disjoint lane sets, in a fixed order.
__device__ __forceinline__ Welford wave_welford(Welford w) {
  w = welford_merge(w, welford_dpp<kDppQuadXor1>(w));
  w = welford_merge(w, welford_dpp<kDppQuadXor2>(w));
  w = welford_merge(w, welford_dpp<kDppRowRor4>(w));
  w = welford_merge(w, welford_dpp<kDppRowRor8>(w));
  return welford_merge(welford_merge(welford_lane(w, 0), welford_lane(w, 16)),
                       welford_merge(welford_lane(w, 32), welford_lane(w, 48)));
}

// Host-side BatchNorm plumbing shared by the two code paths
// (batchnorm.hip: split-K; batchnorm_fused.hip: persistent single pass).
//
// Workspace layout (bytes):
//   [0, 16)                      control words of the single-pass path
//   [16, 16 + fused_slot_bytes)  its exchange slots
//   [.., + split_bytes)          Welford partials of the split-K path
constexpr size_t kBnCtlBytes = 16;
constexpr size_t kBnErrorWordOffset = 8;  // ctl[2]: sticky error word of the single-pass path
int64_t bn_fused_groups(int64_t n, int64_t hw);   // workgroups per channel
size_t bn_fused_slot_bytes(int64_t n, int64_t c, int64_t hw);

// Launches the single-pass kernel if the shape, pointers and device allow
// it.  Returns 0 on launch, a hipError_t / HIPO_EINVAL on failure, and -1 if
// the caller should use the split-K path instead.
int bn_fused_launch(const float* x, const float* gamma, const float* beta,
                    float* running_mean, float* running_var, float* y,
                    float* save_mean, float* save_invstd, int64_t n, int64_t c,
                    int64_t hw, float momentum, float eps, int relu,
                    void* workspace, hipStream_t stream);

}  // namespace hipo
