// BatchNorm training forward, fp32 NCHW, single pass over x.
//
// x is read from HBM once: every workgroup keeps its share of a channel in
// registers from the moment it is loaded until it is normalised and stored.
//
// Decomposition.  A channel's N*HW values are N planes of F = HW/4 float4.
// Counted as one index i in [0, N*F) (plane i / F, offset i % F), they are cut
// into G contiguous slabs of S = ceil(N*F / G) float4, one per workgroup; a
// data thread holds up to V float4 of its slab (index s0 + t + u*448).  The
// grid is R*G workgroups, one per CU (R*G <= CU count); workgroup b serves
// slab k = b % G of channels j, j + R, j + 2R, ... (j = b / G), one channel
// per round.
//
// Workgroup = 7 data waves + 1 exchange wave.  Data waves keep two register
// buffers and software-pipeline the rounds:
//     load round r+1 -> barrier (round r's coefficients ready) -> store round
//     r -> statistics of round r+1 -> barrier
// so the next round's loads are in flight while round r's exchange completes
// and its stores drain.  The exchange wave never touches x or y: its waits
// (the hardware vmcnt counter is in order per wave) are only for its own
// small accesses, so polling never stalls behind bulk traffic.
//
// Exchange between the G workgroups of a channel: each publishes its
// (count, mean, M2) as three 64-bit words {tag, value} with relaxed
// agent-scope atomic stores (a single word needs no ordering, so no L2
// write-back is issued); lane kk of the exchange wave polls partner kk's
// words until all carry this launch's tag, the wave votes with a ballot, and
// the G triples are merged in fp64 in a fixed order -- every workgroup of the
// channel computes identical coefficients.  tag = epoch + 1; the last
// workgroup to finish advances the epoch and clears the completion counter,
// so the next launch starts from a clean state.  Waits are bounded
// (spin_limit polls per workgroup in total); a timed-out wait sets the
// sticky error word and poisons that channel's outputs with NaN, and the
// kernel still exits.
//
// Per-thread statistics are one pass shifted by the thread's first value
// (sums of x - K and (x - K)^2, accumulated as the loads land), then Chan
// merges across the wave (DPP), the workgroup (LDS) and the G slabs (fp64).
//
// Requirements (checked on the host, else the split-K path is used): HW % 4
// == 0, 16-byte aligned x and y, x under 4 GiB (32-bit byte offsets from a
// uniform base), G <= 64, rounds <= 64, and an occupancy of one 512-thread
// workgroup per CU.  All R*G workgroups must be resident at once: the grid
// never exceeds the CU count.
//
// HBM-bound.  Algorithmic bytes: 8 per element (x read once, y written once)
// + O(C).
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "welford.h"

namespace hipo {
namespace {

constexpr int kDataThreads = 448;  // 7 data waves
constexpr int kDataWaves = kDataThreads / kWave;
constexpr int kThreads = kDataThreads + kWave;
constexpr int kFullV = 28;          // float4 per data thread, exact slabs
constexpr int kMaskedV = 24;        // largest masked slab that fits in VGPRs
constexpr uint32_t kSpinLimit = 1u << 20;

struct FusedGeom {
  int C;           // channels
  int F;           // float4 per plane (HW / 4)
  int G;           // workgroups (slabs) per channel
  int R;           // channels per round
  int rounds;
  uint32_t NF;     // float4 per channel (N * F)
  uint32_t S;      // float4 per slab
  uint32_t magic;  // i / F == (i * magic) >> shift for i < 2^31
  int shift;
};

struct FusedArgs {
  const float* gamma;
  const float* beta;
  float* running_mean;
  float* running_var;
  float* save_mean;
  float* save_invstd;
  uint32_t* ctl;     // [0] completion count, [1] epoch, [2] sticky error
  uint64_t* slots;   // [C][G][3] tagged (count, mean, M2)
  float momentum;
  float eps;
  uint32_t spin_limit;
  uint32_t wait_tag_skew;  // 0; 1 only under failure injection (see launch)
  uint32_t copy;           // 1: the hold-copy yardstick (no exchange, y = x)
};

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  // Keeps the compiler from hoisting per-thread index math out of the round
  // loop (it would hold V addresses live across the whole kernel).
  __asm__ volatile("" : "+v"(v));
  return v;
}

struct Pos {
  uint32_t n, off;  // plane, float4 offset in the plane
};

__device__ __forceinline__ Pos pos_of(uint32_t i, const FusedGeom& g) {
  const uint32_t n =
      static_cast<uint32_t>((static_cast<uint64_t>(i) * g.magic) >> g.shift);
  return Pos{n, i - n * static_cast<uint32_t>(g.F)};
}

// Advance by kDataThreads float4 (qk whole planes + rk).
__device__ __forceinline__ void advance(Pos& p, uint32_t F, uint32_t qk,
                                        uint32_t rk) {
  p.off += rk;
  p.n += qk;
  if (p.off >= F) {
    p.off -= F;
    ++p.n;
  }
}

// Float4 of this thread's part of the slab [s0, s1) that are in bounds: u <
// valid_count holds element s0 + tid + u * kDataThreads.
template <int V>
__device__ __forceinline__ int valid_count(uint32_t i0, uint32_t s1) {
  if (i0 >= s1) return 0;
  const uint32_t nv = (s1 - i0 + kDataThreads - 1) / kDataThreads;
  return nv < V ? static_cast<int>(nv) : V;
}

template <int V, bool FULL>
__device__ __forceinline__ void load_slab(const f32x4_t* __restrict__ x,
                                          const FusedGeom& g, int c,
                                          uint32_t s0, uint32_t s1, int tid,
                                          f32x4_t (&v)[V]) {
  const uint32_t F = g.F, qk = kDataThreads / F, rk = kDataThreads % F;
  const uint32_t cF = static_cast<uint32_t>(c) * F;
  const uint32_t CF = static_cast<uint32_t>(g.C) * F;
  const uint32_t i0 = opaque(s0 + tid);
  const int nv = FULL ? V : valid_count<V>(i0, s1);
  Pos p = pos_of(i0, g);
  // Past the slab end a thread re-reads its own first float4 (or the
  // channel's first one if it has none); slab_stats subtracts the copies
  // and store_slab skips them.
  const uint32_t e_first = nv > 0 ? p.n * CF + cF + p.off : cF;
#pragma unroll
  for (int u = 0; u < V; ++u) {
    uint32_t e4 = p.n * CF + cF + p.off;
    if (!FULL) e4 = u < nv ? e4 : e_first;
    v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(
        reinterpret_cast<const char*>(x) + (e4 << 4)));
    advance(p, F, qk, rk);
  }
}

template <int V, bool FULL>
__device__ __forceinline__ Welford slab_stats(const f32x4_t (&v)[V],
                                              uint32_t s0, uint32_t s1,
                                              int tid) {
  const int nv = FULL ? V : valid_count<V>(opaque(s0 + tid), s1);
  const float K = v[0].x;
  float a1 = 0.f, a2 = 0.f, b1 = 0.f, b2 = 0.f;
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const float d0 = v[u].x - K, d1 = v[u].y - K;
    const float d2 = v[u].z - K, d3 = v[u].w - K;
    a1 += d0 + d1;
    b1 += d2 + d3;
    a2 = __builtin_fmaf(d0, d0, a2);
    a2 = __builtin_fmaf(d1, d1, a2);
    b2 = __builtin_fmaf(d2, d2, b2);
    b2 = __builtin_fmaf(d3, d3, b2);
  }
  float s1sum = a1 + b1, s2sum = a2 + b2;
  if (!FULL) {
    // Remove the V - nv copies of v[0] (d0 of v[0] is exactly 0).  No early
    // exit for nv == 0: a branch here costs registers across the loop.
    const float e1 = v[0].y - K, e2 = v[0].z - K, e3 = v[0].w - K;
    const float dup = static_cast<float>(V - nv);
    s1sum -= dup * ((e1 + e2) + e3);
    s2sum -= dup * (__builtin_fmaf(e1, e1, e2 * e2) + e3 * e3);
  }
  const float n = 4.f * static_cast<float>(nv);
  const float dm = n > 0.f ? s1sum / n : 0.f;
  // maximum (not fmaxf) keeps a NaN from the data.
  const float m2 = __builtin_elementwise_maximum(s2sum - s1sum * dm, 0.f);
  return Welford{n, n > 0.f ? K + dm : 0.f, n > 0.f ? m2 : 0.f};
}

template <int V, bool FULL, bool RELU>
__device__ __forceinline__ void store_slab(f32x4_t* __restrict__ y,
                                           const FusedGeom& g, int c,
                                           uint32_t s0, uint32_t s1, int tid,
                                           const f32x4_t (&v)[V], float alpha,
                                           float shift) {
  const uint32_t F = g.F, qk = kDataThreads / F, rk = kDataThreads % F;
  const uint32_t cF = static_cast<uint32_t>(c) * F;
  const uint32_t CF = static_cast<uint32_t>(g.C) * F;
  const uint32_t i1 = opaque(s0 + tid);
  const int nv = FULL ? V : valid_count<V>(i1, s1);
  Pos p = pos_of(i1, g);
#pragma unroll
  for (int u = 0; u < V; ++u) {
    f32x4_t o;
    o.x = __builtin_fmaf(v[u].x, alpha, shift);
    o.y = __builtin_fmaf(v[u].y, alpha, shift);
    o.z = __builtin_fmaf(v[u].z, alpha, shift);
    o.w = __builtin_fmaf(v[u].w, alpha, shift);
    if (RELU) {  // IEEE maximum: NaN stays NaN, as torch.relu
      o.x = __builtin_elementwise_maximum(o.x, 0.f);
      o.y = __builtin_elementwise_maximum(o.y, 0.f);
      o.z = __builtin_elementwise_maximum(o.z, 0.f);
      o.w = __builtin_elementwise_maximum(o.w, 0.f);
    }
    const uint32_t e4 = p.n * CF + cF + p.off;
    if (FULL || u < nv)
      __builtin_nontemporal_store(
          o, reinterpret_cast<f32x4_t*>(reinterpret_cast<char*>(y) + (e4 << 4)));
    advance(p, F, qk, rk);
  }
}

__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ __forceinline__ float lane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ void put_tagged(uint64_t* slot, float v, uint32_t tag) {
  __hip_atomic_store(slot, (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exchange wave, lane 0: merge the data waves' triples, publish slab k of
// channel c.
__device__ __forceinline__ void publish(const Welford* wp, const FusedArgs& a,
                                        const FusedGeom& g, int c, int k,
                                        uint32_t tag) {
  Welford t = wp[0];
  for (int i = 1; i < kDataWaves; ++i) t = welford_merge(t, wp[i]);
  uint64_t* s = a.slots + (static_cast<int64_t>(c) * g.G + k) * 3;
  put_tagged(s + 0, t.n, tag);
  put_tagged(s + 1, t.mean, tag);
  put_tagged(s + 2, t.m2, tag);
}

// Per-round channel parameters, prefetched once: lane r holds round r's.
struct ChannelParams {
  float gamma, beta, rmean, rvar;
};

// Exchange wave (all lanes): wait for the G slabs of channel c, merge them,
// write the normalisation coefficients to LDS; slab 0 also writes
// save_mean / save_invstd and the running statistics.
// `budget` is the workgroup's remaining poll count over all rounds, so a
// partner that never arrives costs one bounded wait per kernel, not one per
// round.
__device__ __forceinline__ void finish_channel(float* coef, const FusedArgs& a,
                                               const FusedGeom& g, int c, int k,
                                               int r, uint32_t tag,
                                               const ChannelParams& cp,
                                               int lane, uint32_t& budget) {
  const bool mine = lane < g.G;
  const uint32_t want = tag + a.wait_tag_skew;
  const uint64_t* s =
      a.slots + (static_cast<int64_t>(c) * g.G + (mine ? lane : 0)) * 3;
  uint64_t w0 = 0, w1 = 0, w2 = 0;
  bool ok = true;
  while (true) {
    if (mine) {
      w0 = __hip_atomic_load(s + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      w1 = __hip_atomic_load(s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      w2 = __hip_atomic_load(s + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool have = !mine || (static_cast<uint32_t>(w0 >> 32) == want &&
                                static_cast<uint32_t>(w1 >> 32) == want &&
                                static_cast<uint32_t>(w2 >> 32) == want);
    if (__builtin_amdgcn_ballot_w64(!have) == 0) break;
    if (budget == 0) {
      ok = false;
      break;
    }
    --budget;
    __builtin_amdgcn_s_sleep(1);
  }
  const float fn = __uint_as_float(static_cast<uint32_t>(w0));
  const float fm = __uint_as_float(static_cast<uint32_t>(w1));
  const float fq = __uint_as_float(static_cast<uint32_t>(w2));
  double count = 0.0, mean = 0.0, m2 = 0.0;
  for (int kk = 0; kk < g.G; ++kk) {
    const double nb = lane_f32(fn, kk), mb = lane_f32(fm, kk), qb = lane_f32(fq, kk);
    const double tot = count + nb;
    if (tot == 0.0) continue;
    const double d = mb - mean;
    mean += d * (nb / tot);
    m2 += qb + d * d * count * (nb / tot);
    count = tot;
  }
  const float meanf = static_cast<float>(mean);
  const float var = static_cast<float>(m2 / count);
  float invstd = 1.0f / __builtin_sqrtf(var + a.eps);
  if (!ok) invstd = __builtin_nanf("");
  const float alpha = invstd * lane_f32(cp.gamma, r);
  if (lane == 0) {
    if (!ok) __hip_atomic_store(a.ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    coef[0] = alpha;
    coef[1] = lane_f32(cp.beta, r) - meanf * alpha;
    if (k == 0) {
      // A timed-out wait merged slots of an older launch: every statistic
      // derived from them, the persistent running statistics included, is
      // poisoned with NaN rather than written as plausible finite values.
      const double unbiased = count > 1.0 ? m2 / (count - 1.0) : __builtin_nan("");
      const double mom = a.momentum;
      const float rm = static_cast<float>(mom * mean + (1.0 - mom) * lane_f32(cp.rmean, r));
      const float rv =
          static_cast<float>(mom * unbiased + (1.0 - mom) * lane_f32(cp.rvar, r));
      a.save_mean[c] = ok ? meanf : __builtin_nanf("");
      a.save_invstd[c] = invstd;
      a.running_mean[c] = ok ? rm : __builtin_nanf("");
      a.running_var[c] = ok ? rv : __builtin_nanf("");
    }
  }
}

// a.copy (the hold-copy yardstick, hipo_hold_copy_f32; uniform): the same
// slabs, rounds, register buffers, loads, per-thread statistics (which wait
// for each round's loads), barriers and stores, with no exchange between
// workgroups: the exchange wave sets the coefficients to alpha = 1, shift =
// -0, so the stored fma(x, 1, -0) is x itself (signed zeros included; a
// signalling NaN comes out quiet).  A runtime flag, not a template
// parameter, so the data waves run the kernel's own code.
template <int V, bool FULL, bool RELU>
__global__ __launch_bounds__(kThreads) void bn_train_fused(
    const f32x4_t* __restrict__ x, f32x4_t* __restrict__ y, FusedArgs a,
    FusedGeom g) {
  __shared__ Welford wp[kDataWaves];
  __shared__ float coef[2];
  __shared__ uint32_t epoch_s;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  if (!a.copy && tid == kDataThreads)
    epoch_s = __hip_atomic_load(a.ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  block_sync();
  const uint32_t epoch = epoch_s;
  const uint32_t tag = epoch + 1;
  const int j = blockIdx.x / g.G;
  const int k = blockIdx.x - j * g.G;
  const uint32_t s0 = static_cast<uint32_t>(k) * g.S;
  const uint32_t s1 = min(s0 + g.S, g.NF);
  const int nr = j < g.C ? min(g.rounds, (g.C - j + g.R - 1) / g.R) : 0;
  auto chan = [&](int r) { return r * g.R + j; };

  if (a.copy && nr > 0 && wave == kDataWaves) {
    // ---- the exchange wave's barriers, nothing exchanged
    if (lane == 0) {
      coef[0] = 1.0f;
      coef[1] = -0.0f;
    }
    block_sync();
    for (int r = 0; r < nr; ++r) {
      block_sync();
      if (r + 1 < nr) block_sync();
    }
  } else if (nr > 0 && wave == kDataWaves) {
    // ---- exchange wave
    ChannelParams cp{0.f, 0.f, 0.f, 0.f};
    if (lane < nr) {
      const int c = chan(lane);
      cp.gamma = a.gamma[c];
      cp.beta = a.beta[c];
      if (k == 0) {
        cp.rmean = a.running_mean[c];
        cp.rvar = a.running_var[c];
      }
    }
    uint32_t budget = a.spin_limit;
    block_sync();  // round 0's statistics are in LDS
    if (lane == 0) publish(wp, a, g, chan(0), k, tag);
    for (int r = 0; r < nr; ++r) {
      finish_channel(coef, a, g, chan(r), k, r, tag, cp, lane, budget);
      block_sync();  // coefficients of round r ready
      if (r + 1 < nr) {
        block_sync();  // statistics of round r+1 ready
        if (lane == 0) publish(wp, a, g, chan(r + 1), k, tag);
      }
    }
  } else if (nr > 0) {
    // ---- data waves
    f32x4_t bufA[V], bufB[V];
    auto wave_part = [&](Welford w) {
      w = wave_welford(w);
      if (lane == 0) wp[wave] = w;
    };
    load_slab<V, FULL>(x, g, chan(0), s0, s1, tid, bufA);
    wave_part(slab_stats<V, FULL>(bufA, s0, s1, tid));
    block_sync();
    // Rounds with a successor load unconditionally (a conditional load
    // followed by a conditional consumer would leave the loads pending
    // across the loop edge for the hardware-wait pass); the last round is
    // peeled.
#define HIPO_BN_ROUND(CUR, NXT, RND)                                           \
    {                                                                          \
      load_slab<V, FULL>(x, g, chan((RND) + 1), s0, s1, tid, NXT);             \
      block_sync();                                                            \
      store_slab<V, FULL, RELU>(y, g, chan(RND), s0, s1, tid, CUR, coef[0],    \
                                coef[1]);                                      \
      wave_part(slab_stats<V, FULL>(NXT, s0, s1, tid));                        \
      block_sync();                                                            \
    }
#define HIPO_BN_LAST(CUR, RND)                                                 \
    {                                                                          \
      block_sync();                                                            \
      store_slab<V, FULL, RELU>(y, g, chan(RND), s0, s1, tid, CUR, coef[0],    \
                                coef[1]);                                      \
    }
    int r = 0;
    bool last_in_b = false;
    while (r + 1 < nr) {
      HIPO_BN_ROUND(bufA, bufB, r);
      ++r;
      if (r + 1 >= nr) {
        last_in_b = true;
        break;
      }
      HIPO_BN_ROUND(bufB, bufA, r);
      ++r;
    }
    if (last_in_b) {
      HIPO_BN_LAST(bufB, r);
    } else {
      HIPO_BN_LAST(bufA, r);
    }
#undef HIPO_BN_ROUND
#undef HIPO_BN_LAST
  }
  if (!a.copy && tid == kDataThreads) {
    // The last workgroup out resets the completion count and opens the next
    // epoch; every workgroup has read this launch's epoch by then.
    const uint32_t done =
        __hip_atomic_fetch_add(a.ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1) {
      __hip_atomic_store(a.ctl, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctl + 1, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

using FusedKernel = void (*)(const f32x4_t*, f32x4_t*, FusedArgs, FusedGeom);

// Instantiations: exact slabs of 28 float4 per thread, and masked slabs of
// up to 16 / 24 float4 (two buffers of 28 masked float4 would not fit in
// 256 VGPRs).  Channels this kernel is given hold more than 16384 values
// (smaller ones take the register-held one-launch kernel), so a masked slab
// has at least 10 float4 per thread.
struct Variant {
  int v;
  bool full;
  FusedKernel relu, plain;
};
const Variant kVariants[] = {
    {28, true, bn_train_fused<28, true, true>, bn_train_fused<28, true, false>},
    {16, false, bn_train_fused<16, false, true>, bn_train_fused<16, false, false>},
    {24, false, bn_train_fused<24, false, true>, bn_train_fused<24, false, false>},
};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

// Whether one workgroup of each instantiation fits on a CU, per device.
// kind: 0 plain (also the hold copy), 1 ReLU.
FusedKernel variant_kernel(int variant, int kind) {
  const Variant& vt = kVariants[variant];
  return kind == 1 ? vt.relu : vt.plain;
}

bool resident(int device, int variant, int kind) {
  static std::mutex mu;
  static std::vector<int8_t> cache;  // [device][variant][kind]: -1 unknown
  std::lock_guard<std::mutex> lock(mu);
  const size_t idx = (static_cast<size_t>(device) * kNumVariants + variant) * 2 + kind;
  if (cache.size() <= idx) cache.resize(idx + 1, -1);
  if (cache[idx] < 0) {
    int blocks = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &blocks, reinterpret_cast<const void*>(variant_kernel(variant, kind)), kThreads, 0);
    cache[idx] = (e == hipSuccess && blocks >= 1) ? 1 : 0;
    if (e != hipSuccess) (void)hipGetLastError();
  }
  return cache[idx] == 1;
}

void division_magic(uint32_t d, uint32_t& magic, int& shift) {
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  shift = 31 + l;
  magic = static_cast<uint32_t>(((uint64_t{1} << shift) + d - 1) / d);
}

}  // namespace

// Slabs per channel: exact 28-float4-per-thread slabs when N*F is a multiple
// of that slab, else masked slabs of at most kMaskedV per thread.
int64_t bn_fused_groups(int64_t n, int64_t hw) {
  const int64_t nf = n * (hw / 4);
  if (nf <= 0) return 0;
  const int64_t full = int64_t{kFullV} * kDataThreads;
  if (nf % full == 0) return nf / full;
  const int64_t cap = int64_t{kMaskedV} * kDataThreads;
  return (nf + cap - 1) / cap;
}

size_t bn_fused_slot_bytes(int64_t n, int64_t c, int64_t hw) {
  if (hw % 4 != 0) return 0;
  const int64_t g = bn_fused_groups(n, hw);
  if (g <= 0 || g > 64) return 0;
  return static_cast<size_t>(c * g * 3) * sizeof(uint64_t);
}

namespace {

// Slabs, rounds and instantiation of the single-pass geometry for x / y
// [n, c, hw] fp32; false when the shape or the device falls outside it.
bool fused_plan(const float* x, const float* y, int64_t n, int64_t c, int64_t hw, int kind,
                FusedGeom& g, int& variant, int64_t& grid) {
  if (hw % 4 != 0 || !aligned16(x) || !aligned16(y)) return false;
  const int64_t F = hw / 4;
  const int64_t nf = n * F;
  if (n * c * hw * 4 >= (int64_t{1} << 32) || nf >= (int64_t{1} << 31)) return false;
  const DeviceInfo* dev = device_info();
  if (!dev) return false;
  const int64_t G = bn_fused_groups(n, hw);
  if (G < 1 || G > 64 || G > dev->cu_count) return false;
  const int64_t R = std::min<int64_t>(c, dev->cu_count / G);
  const int64_t rounds = (c + R - 1) / R;
  if (rounds > 64) return false;
  const int64_t S = (nf + G - 1) / G;
  const int64_t per_thread = (S + kDataThreads - 1) / kDataThreads;
  variant = -1;
  if (S == int64_t{kFullV} * kDataThreads && G * S == nf) {
    variant = 0;
  } else {
    for (int i = 1; i < kNumVariants; ++i) {
      if (kVariants[i].v >= per_thread) {
        variant = i;
        break;
      }
    }
  }
  if (variant < 0 || !resident(dev->device, variant, kind)) return false;
  g.C = static_cast<int>(c);
  g.F = static_cast<int>(F);
  g.G = static_cast<int>(G);
  g.R = static_cast<int>(R);
  g.rounds = static_cast<int>(rounds);
  g.NF = static_cast<uint32_t>(nf);
  g.S = static_cast<uint32_t>(S);
  division_magic(static_cast<uint32_t>(F), g.magic, g.shift);
  grid = R * G;
  return true;
}

}  // namespace

int bn_fused_launch(const float* x, const float* gamma, const float* beta,
                    float* running_mean, float* running_var, float* y,
                    float* save_mean, float* save_invstd, int64_t n, int64_t c,
                    int64_t hw, float momentum, float eps, int relu,
                    void* workspace, hipStream_t stream) {
  if (!aligned16(workspace)) return -1;
  FusedGeom g;
  int variant = -1;
  int64_t grid = 0;
  if (!fused_plan(x, y, n, c, hw, relu ? 1 : 0, g, variant, grid)) return -1;

  char* ws = static_cast<char*>(workspace);
  FusedArgs a;
  a.gamma = gamma;
  a.beta = beta;
  a.running_mean = running_mean;
  a.running_var = running_var;
  a.save_mean = save_mean;
  a.save_invstd = save_invstd;
  a.ctl = reinterpret_cast<uint32_t*>(ws);
  a.slots = reinterpret_cast<uint64_t*>(ws + kBnCtlBytes);
  a.momentum = momentum;
  a.eps = eps;
  // Failure injection, for the tests of the timeout path: with
  // HIPO_TEST_FORCE_BN_TIMEOUT set in the environment, every exchange wait
  // looks for a tag no workgroup publishes and gives up after a few polls,
  // so the kernel takes its timeout path (error word, NaN outputs) and still
  // exits normally.  The launch epoch advances as usual.
  const bool force_timeout = getenv("HIPO_TEST_FORCE_BN_TIMEOUT") != nullptr;
  a.spin_limit = force_timeout ? 8u : kSpinLimit;
  a.wait_tag_skew = force_timeout ? 1u : 0u;
  a.copy = 0;

  const FusedKernel kernel = variant_kernel(variant, relu ? 1 : 0);
  kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream>>>(
      reinterpret_cast<const f32x4_t*>(x), reinterpret_cast<f32x4_t*>(y), a, g);
  return check_launch("batchnorm_train_fwd_f32 (single pass)");
}

int bn_hold_copy_launch(const float* x, float* y, int64_t n, int64_t c, int64_t hw,
                        hipStream_t stream) {
  FusedGeom g;
  int variant = -1;
  int64_t grid = 0;
  if (!fused_plan(x, y, n, c, hw, 0, g, variant, grid)) return -1;
  FusedArgs a{};  // the copy reads no parameters and exchanges nothing
  a.copy = 1;
  variant_kernel(variant, 0)<<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream>>>(
      reinterpret_cast<const f32x4_t*>(x), reinterpret_cast<f32x4_t*>(y), a, g);
  return check_launch("hold_copy_f32");
}

}  // namespace hipo

extern "C" int hipo_hold_copy_f32(const float* x, float* y, int64_t n, int64_t c, int64_t hw,
                                  hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n > 0 && c > 0 && hw > 0, "hold_copy: sizes must be positive");
  HIPO_REQUIRE(x && y, "hold_copy: null pointer");
  const int rc = bn_hold_copy_launch(x, y, n, c, hw, stream);
  HIPO_REQUIRE(rc >= 0,
               "hold_copy: [%lld, %lld, %lld] is outside the single-pass BatchNorm geometry "
               "(H*W a multiple of 4, 16-byte aligned, at most 64 slabs and 64 rounds)",
               (long long)n, (long long)c, (long long)hw);
  return rc;
}
