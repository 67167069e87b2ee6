// BatchNorm training forward on bf16 activations (fp32 statistics) with the
// epilogues of two corpus families:
//   * channels-last x [N, C, H, W] (physical [N*H*W, C]) -> activation ->
//     zero pad of the bottom / right border, channels-last output
//     (reference repros/canonical/var_mean_ceb5c315290a: SiLU, pad 1);
//   * NCHW x [N, C, H, W] -> activation -> mean over H, W -> [N, C]
//     (reference repros/canonical/var_mean_mean_19ffdb35cc67: ReLU).
// Semantics (the eager graphs' op order):
//   mean, var = var_mean(fp32(x), [0, 2, 3], correction 0)
//   save_rstd = 1 / sqrt(var + eps)
//   y = act(bf16(((x - mean) * save_rstd) * gamma + beta))   (fp32 ops)
//   running_mean = mean * momentum + running_mean * (1 - momentum)
//   running_var  = (var * var_scale) * momentum + running_var * (1 - momentum)
// var_scale is the graph's Bessel constant (N/(N-1) of the shape the graph
// was captured at), passed through unchanged.
//
// Three launches (two for NCHW), no atomics, deterministic:
//   1. partial statistics per slice of the reduction axis -> workspace
//      (mean, M2) per (slice, channel);
//   2. a per-channel merge of the slices in fp64 (a fixed order) that writes
//      save_mean, save_rstd and the running statistics -- its own launch for
//      channels-last; folded into the epilogue's workgroups for NCHW, whose
//      channels each workgroup merges itself;
//   3. the normalise + activation pass (padded store / spatial mean).
// HBM-bound: x is read twice and the output written once.  NCHW shapes whose
// channels fit a workgroup's registers (N * HW <= 8192, HW <= 64) take one
// launch instead (bn_nchw_channels): x read once, no workspace.
#include <algorithm>

#include "hipo_common.h"

namespace hipo {
namespace {

constexpr int kMaxThreads = 1024;

enum { kActNone = 0, kActRelu = 1, kActSilu = 2 };

// SiLU(t) = t / (1 + e^-t) of a bf16 value t, in fp32; callers round it to
// bf16.  That rounding gives the correctly rounded SiLU of every bf16 t,
// and -0 where e^-t overflows fp32 (t < -88.72), as eager's expf does.
//
// Common inputs (t > -87): t * rcp(1 + 2^(t * -log2 e)), with the hardware
// exp2 (v_exp_f32) and reciprocal (v_rcp_f32) -- 3 VALU and 2 transcendental
// instructions where the accurate form below takes ~18.  Over all bf16
// t > -87 this rounds to the correctly rounded SiLU except at t = 5.9375,
// whose exact SiLU lies 1.18 fp32 ulps below the bf16 midpoint 5.921875 and
// which one select patches (to 5.90625).  The GPU tests run all 65536 bf16
// inputs through the kernels and compare bit for bit with mpmath; the GPU's
// exp2 and rcp are deterministic and the domain is finite, so that is the
// proof.  At -88.5 <= t <= -87.5 the reciprocal's result is an fp32
// denormal, which the hardware reciprocal flushes to zero.
//
// Rare inputs (t <= -87, NaN): the accurate form, the extended-precision
// exp_f32 and an IEEE division, correctly rounded there too.
constexpr float kSiluNegLog2e = -1.4426950408889634f;
constexpr float kSiluFastMin = -87.0f;

__device__ __forceinline__ float silu_fast(float t) {
  const float y = t * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(t * kSiluNegLog2e));
  return t == 5.9375f ? 5.90625f : y;
}

__device__ __forceinline__ float silu_accurate(float t) {
  return t / (1.f + exp_f32(exp_domain(-t)));
}

__device__ __forceinline__ float silu_of_bf16(float t) {
  return __builtin_expect(t > kSiluFastMin, 1) ? silu_fast(t) : silu_accurate(t);
}

// bf16(((x - mean) * rstd) * gamma + beta), fp32 ops in the eager order (no
// contraction): the activation's input.
__device__ __forceinline__ float bn_affine(float x, float mean, float rstd, float g, float b) {
  const float y = __fmul_rn(__fsub_rn(x, mean), rstd);
  return round_bf16(__fadd_rn(__fmul_rn(y, g), b));
}

// act(bn_affine(...)); callers round the result to bf16 (eager's activation
// output) before storing or summing it.  (A correctly rounded bf16 SiLU
// table staged in LDS, like the GELU kernels', measured 2-5 % slower in the
// channels-last epilogue than the accurate form silu_of_bf16 uses for rare
// inputs.)
__device__ __forceinline__ float bn_act(float x, float mean, float rstd, float g, float b,
                                        int act) {
  float y = bn_affine(x, mean, rstd, g, b);
  if (act == kActRelu) {
    y = y < 0.f ? 0.f : y;
  } else if (act == kActSilu) {
    y = silu_of_bf16(y);
  }
  return y;
}

// The activation of 8 values with the activation known at compile time, so
// the 8 evaluations interleave: SiLU takes the fast form for all 8 and
// redoes them with silu_of_bf16 only when one of them is rare (t <= -87 or
// NaN; the comparison is false for NaN).
template <int ACT>
__device__ __forceinline__ void bn_act_x8(float (&y)[8]) {
  if constexpr (ACT == kActRelu) {
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = y[e] < 0.f ? 0.f : y[e];
  } else if constexpr (ACT == kActSilu) {
    float s[8];
    bool rare = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[e] = silu_fast(y[e]);
      rare |= !(y[e] > kSiluFastMin);
    }
    if (__builtin_expect(rare, 0)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = silu_of_bf16(y[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = s[e];
  }
}

// Chan's pairwise merge of (count, mean, M2) partials: (n, mean, m2) <-
// (n, mean, m2) + (nb, meanb, m2b).
template <typename T>
__device__ __forceinline__ void chan_merge(T& n, T& mean, T& m2, T nb, T meanb, T m2b) {
  if (nb == T(0)) return;
  const T nn = n + nb;
  const T d = meanb - mean;
  const T f = nb / nn;
  mean = mean + d * f;
  m2 = m2 + m2b + d * d * n * f;
  n = nn;
}

__device__ __forceinline__ void unpack8(const u32x4_t v, float (&f)[8]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f[2 * d] = bf16lo(v[d]);
    f[2 * d + 1] = bf16hi(v[d]);
  }
}

// ---------------------------------------------------------------------------
// Channels-last: x is [M, C] rows (M = N*H*W), G = C / 8 groups of 16 bytes.
// A workgroup of T threads (T a multiple of G) covers T / G whole rows per
// access instruction; thread t owns group t % G.  x is read twice (the
// statistics pass, then the epilogue) with ordinary cached loads, and the
// epilogue walks the rows in reverse: it starts on the rows the statistics
// pass read last, the likeliest to be still in the 256 MB Infinity Cache
// (all of x when it fits there).
// ---------------------------------------------------------------------------

// Workgroup s reduces rows [s*L, min(M, (s+1)*L)): sums of (x - shift) and
// (x - shift)^2 per channel, shift = the slice's first row, with kStatUnroll
// loads in flight per thread; the R = T / G row partials of a group are added
// by a fixed-order halving tree in LDS (R is a power of two) and turned into
// (mean, M2) for the slice.
constexpr int kStatUnroll = 8;
__global__ __launch_bounds__(kMaxThreads) void bn_nhwc_partial(
    const uint16_t* __restrict__ x, float2* __restrict__ part, int64_t M, int64_t C, int G,
    int64_t L) {
  extern __shared__ float lds[];  // [T / 2][16]
  const int T = blockDim.x;
  const int t = threadIdx.x;
  const int g = t % G;
  const int r = t / G;
  const int R = T / G;
  const int64_t s = blockIdx.x;
  const int64_t p0 = s * L;
  const int64_t p1 = std::min<int64_t>(M, p0 + L);
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x) + g;
  const int64_t G64 = G;

  const u32x4_t shv = xv[p0 * G64];
  float shift[8];
  unpack8(shv, shift);
  float s1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float s2[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t p = p0 + r; p < p1; p += static_cast<int64_t>(R) * kStatUnroll) {
    u32x4_t v[kStatUnroll];
#pragma unroll
    for (int u = 0; u < kStatUnroll; ++u) {
      // Rows past the slice re-read its first row and count as the shift
      // (a zero deviation).
      const int64_t pu = p + static_cast<int64_t>(u) * R;
      v[u] = xv[(pu < p1 ? pu : p0) * G64];
      if (pu >= p1) v[u] = shv;
    }
#pragma unroll
    for (int u = 0; u < kStatUnroll; ++u) {
      float f[8];
      unpack8(v[u], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = f[e] - shift[e];
        s1[e] += d;
        s2[e] = __builtin_fmaf(d, d, s2[e]);
      }
    }
  }
  // At each level rows [half, 2 half) store to slot (r - half) * G + g and
  // rows [0, half) add the slot of row r + half of their group.
  for (int half = R / 2; half > 0; half /= 2) {
    if (r >= half && r < 2 * half) {
      float* slot = lds + ((r - half) * G + g) * 16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        slot[e] = s1[e];
        slot[8 + e] = s2[e];
      }
    }
    __syncthreads();
    if (r < half) {
      const float* slot = lds + (r * G + g) * 16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s1[e] += slot[e];
        s2[e] += slot[8 + e];
      }
    }
    __syncthreads();
  }
  if (t >= G) return;
  const float n = static_cast<float>(p1 - p0);
  const int64_t S = gridDim.x;
  float2* dst = part + (8 * g) * S + s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float d = s1[e] / n;
    dst[e * S] = make_float2(shift[e] + d, fmaxf(s2[e] - s1[e] * d, 0.f));
  }
}

// Output row o = (n, ho, wo) of the padded [N, Ho, Wo, C] tensor: the
// normalised, activated x row (n, ho, wo) when ho < H and wo < W, else zeros.
// Workgroup b writes rows [b'*R*kApplyUnroll, (b'+1)*R*kApplyUnroll),
// b' = gridDim.x - 1 - b (reverse order, see above).
constexpr int kApplyUnroll = 4;
template <int ACT>
__global__ __launch_bounds__(kMaxThreads) void bn_nhwc_apply_pad(
    const uint16_t* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, uint16_t* __restrict__ out, uint32_t rows_out, uint32_t H,
    uint32_t W, uint32_t Ho, uint32_t Wo, DivMagic image_div, DivMagic row_div, int G) {
  const int T = blockDim.x;
  const int t = threadIdx.x;
  const int g = t % G;
  const int r = t / G;
  const int R = T / G;
  float m[8], rs[8], ga[8], be[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    m[e] = mean[8 * g + e];
    rs[e] = rstd[8 * g + e];
    ga[e] = gamma[8 * g + e];
    be[e] = beta[8 * g + e];
  }
  const u32x4_t* xv = reinterpret_cast<const u32x4_t*>(x) + g;
  u32x4_t* ov = reinterpret_cast<u32x4_t*>(out) + g;
  const uint32_t o0 = (gridDim.x - 1 - blockIdx.x) * static_cast<uint32_t>(R * kApplyUnroll) + r;
  const int64_t G64 = G;
  u32x4_t v[kApplyUnroll];
  bool inside[kApplyUnroll];
#pragma unroll
  for (int u = 0; u < kApplyUnroll; ++u) {
    const uint32_t o = o0 + static_cast<uint32_t>(u * R);
    const uint32_t img = div_by(o, image_div);  // o / (Ho Wo), the load depends on it
    const uint32_t rem = o - img * (Ho * Wo);
    const uint32_t ho = div_by(rem, row_div);   // rem / Wo
    const uint32_t wo = rem - ho * Wo;
    inside[u] = o < rows_out && ho < H && wo < W;
    // Padding and rows past the end read row 0 (in bounds) and store zeros.
    const int64_t src = inside[u] ? (static_cast<int64_t>(img) * H + ho) * W + wo : 0;
    v[u] = xv[src * G64];
  }
#pragma unroll
  for (int u = 0; u < kApplyUnroll; ++u) {
    const uint32_t o = o0 + static_cast<uint32_t>(u * R);
    if (o >= rows_out) continue;
    float f[8];
    unpack8(v[u], f);
    // Padding: act(0) = 0 for every activation, so the select goes first.
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = inside[u] ? bn_affine(f[e], m[e], rs[e], ga[e], be[e]) : 0.f;
    bn_act_x8<ACT>(f);
    u32x4_t w;
#pragma unroll
    for (int d = 0; d < 4; ++d) w[d] = pack_bf16x2(f[2 * d], f[2 * d + 1]);
    __builtin_nontemporal_store(w, ov + static_cast<int64_t>(o) * G64);
  }
}

// Any C / alignment: one thread per (slice, channel).
__global__ __launch_bounds__(256) void bn_nhwc_partial_scalar(
    const uint16_t* __restrict__ x, float2* __restrict__ part, int64_t M, int64_t C, int64_t L) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int64_t s = blockIdx.y;
  const int64_t p0 = s * L;
  const int64_t p1 = std::min<int64_t>(M, p0 + L);
  const float shift = bf16_to_f32(x[p0 * C + c]);
  float s1 = 0.f, s2 = 0.f;
  for (int64_t p = p0; p < p1; ++p) {
    const float d = bf16_to_f32(x[p * C + c]) - shift;
    s1 += d;
    s2 = __builtin_fmaf(d, d, s2);
  }
  const float n = static_cast<float>(p1 - p0);
  const float d = s1 / n;
  part[c * static_cast<int64_t>(gridDim.y) + s] = make_float2(shift + d, fmaxf(s2 - s1 * d, 0.f));
}

__global__ __launch_bounds__(256) void bn_nhwc_apply_pad_scalar(
    const uint16_t* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, uint16_t* __restrict__ out, int64_t total, int64_t H,
    int64_t W, int64_t Ho, int64_t Wo, int64_t C, int act) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t c = i % C;
  const int64_t o = i / C;
  const int64_t img = o / (Ho * Wo);
  const int64_t rem = o - img * (Ho * Wo);
  const int64_t ho = rem / Wo;
  const int64_t wo = rem - ho * Wo;
  float y = 0.f;
  if (ho < H && wo < W) {
    const float xv = bf16_to_f32(x[((img * H + ho) * W + wo) * C + c]);
    y = bn_act(xv, mean[c], rstd[c], gamma[c], beta[c], act);
  }
  out[i] = static_cast<uint16_t>(pack_bf16x2(y, 0.f) & 0xffffu);
}

// ---------------------------------------------------------------------------
// NCHW, general shapes: a workgroup of kNchwImages waves covers a block of
// 64 channels (lane = channel) of kNchwImages consecutive images (wave =
// image); each lane reads its channel's HW values from memory.
// ---------------------------------------------------------------------------
constexpr int kNchwImages = 4;
constexpr int kNchwChannels = 64;

// What the NCHW epilogue pass needs to merge its channels' slice statistics
// itself (the statistics pass wrote (mean, M2) per (channel, slice of
// kNchwImages images), channel-major).
struct NchwMerge {
  const float2* part;
  int64_t slices;
  float* running_mean;
  float* running_var;
  float* save_mean;
  float* save_rstd;
  float momentum, eps, var_scale;
};

// MODE 0: per (channel, slice of kNchwImages images) partial (mean, M2),
//         exact two-pass statistics of each (image, channel) segment merged
//         over the images in order.
// MODE 1: the workgroup first merges the slice partials of its 64 channels
//         (fp64 sums about the shift m_0, slices strided over the waves, the
//         waves added in order: the same result in every workgroup; the
//         workgroups of the first image group write save_* and the running
//         statistics), then out[n, c] = bf16(sum_hw act(bn(x[n, c, hw])) / HW).
template <int MODE>
__global__ __launch_bounds__(kNchwImages * kWave) void bn_nchw_small_hw(
    const uint16_t* __restrict__ x, float2* __restrict__ part, NchwMerge mg,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    uint16_t* __restrict__ out, int64_t N, int64_t C, int64_t HW, int act) {
  __shared__ float2 stats[kNchwImages][kNchwChannels];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x >> 6;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kNchwChannels;
  const int64_t img = static_cast<int64_t>(blockIdx.y) * kNchwImages + w;
  const int64_t c = c0 + lane;
  const bool img_valid = img < N;
  const bool valid = img_valid && c < C;
  const uint16_t* seg = x + ((img_valid ? img : 0) * C + c0 + lane) * HW;
  if constexpr (MODE == 0) {
    float mu = 0.f, m2 = 0.f;
    if (valid) {
      float sum = 0.f;
      for (int64_t j = 0; j < HW; ++j) sum += bf16_to_f32(seg[j]);
      mu = sum / static_cast<float>(HW);
      for (int64_t j = 0; j < HW; ++j) {
        const float d = bf16_to_f32(seg[j]) - mu;
        m2 = __builtin_fmaf(d, d, m2);
      }
    }
    stats[w][lane] = make_float2(mu, m2);
    __syncthreads();
    if (w == 0 && c < C) {
      float n = 0.f, mm = 0.f, mq = 0.f;
      for (int k = 0; k < kNchwImages; ++k) {
        if (static_cast<int64_t>(blockIdx.y) * kNchwImages + k >= N) break;
        chan_merge(n, mm, mq, static_cast<float>(HW), stats[k][lane].x, stats[k][lane].y);
      }
      part[c * static_cast<int64_t>(gridDim.y) + blockIdx.y] = make_float2(mm, mq);
    }
  } else {
    __shared__ double red[kNchwImages][kNchwChannels][3];
    const float2* pc = mg.part + (c < C ? c : C - 1) * mg.slices;
    const double K = static_cast<double>(pc[0].x);
    {
      double n = 0.0, s1 = 0.0, s2 = 0.0;
      for (int64_t s = w; s < mg.slices; s += kNchwImages) {
        const double cnt = static_cast<double>(
            (std::min<int64_t>(N, (s + 1) * kNchwImages) - s * kNchwImages) * HW);
        const float2 pv = pc[s];
        const double d = static_cast<double>(pv.x) - K;
        n += cnt;
        s1 = __builtin_fma(cnt, d, s1);
        s2 += __builtin_fma(cnt * d, d, static_cast<double>(pv.y));
      }
      red[w][lane][0] = n;
      red[w][lane][1] = s1;
      red[w][lane][2] = s2;
    }
    __syncthreads();
    double n = 0.0, s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int k = 0; k < kNchwImages; ++k) {
      n += red[k][lane][0];
      s1 += red[k][lane][1];
      s2 += red[k][lane][2];
    }
    const double dm = s1 / n;
    const float mc = static_cast<float>(K + dm);
    const float var_f = static_cast<float>(std::max(0.0, s2 - s1 * dm) / n);
    const float rc = 1.0f / __builtin_sqrtf(__fadd_rn(var_f, mg.eps));
    if (blockIdx.y == 0 && w == 0 && c < C) {
      mg.save_mean[c] = mc;
      mg.save_rstd[c] = rc;
      const float keep = 1.0f - mg.momentum;
      mg.running_mean[c] =
          __fadd_rn(__fmul_rn(mc, mg.momentum), __fmul_rn(mg.running_mean[c], keep));
      mg.running_var[c] = __fadd_rn(__fmul_rn(__fmul_rn(var_f, mg.var_scale), mg.momentum),
                                    __fmul_rn(mg.running_var[c], keep));
    }
    if (!valid) return;
    const float gc = gamma[c], bc = beta[c];
    float sum = 0.f;
    for (int64_t j = 0; j < HW; ++j)
      sum += round_bf16(bn_act(bf16_to_f32(seg[j]), mc, rc, gc, bc, act));
    out[img * C + c] = static_cast<uint16_t>(pack_bf16x2(sum / static_cast<float>(HW), 0.f) & 0xffffu);
  }
}

// ---------------------------------------------------------------------------
// NCHW with small planes (C % 8 == 0, HW <= kPlanesMaxHw, x 16-byte
// aligned): a wave covers 8 consecutive channels of the kNchwImages images
// of one slice -- per image, 8 consecutive H x W planes: 16 * HW bytes, a
// whole number of 16-byte vectors whatever HW is.  The wave issues all its
// non-temporal 16-byte loads at once, stages the planes in LDS, and reduces
// each plane over 8 lanes (lane 8r + k takes elements k, k + 8, ... of plane
// r) with a fixed butterfly.  A workgroup holds kPlaneWaves such waves: 32
// channels of one slice.
// MODE 0: each plane's exact two-pass (mean, M2), merged over the slice's
//   images in order -> part[c * slices + s] (the layout of the general path).
// MODE 1: the channel's slices merged in fp64 about the shift m_0 (8 lanes,
//   a fixed order: the same in every wave; the waves of slice 0 write save_*
//   and the running statistics) while the loads are in flight, then
//   out[n, c] = bf16(sum_hw act(bn(x)) / HW).
// ---------------------------------------------------------------------------
constexpr int kPlaneWaves = 4;
constexpr int kPlaneChannels = 8;  // per wave
constexpr int kPlanesMaxHw = 128;

// HWB: plane-size bucket (8, 16, 32, 64 or 128 >= HW): each lane holds
// HWB / 8 values of a plane, and a wave loads at most 4 * HWB / 64 vectors
// per lane, so both loops have fixed trip counts and their loads issue
// together.
template <int MODE, int HWB>
__global__ __launch_bounds__(kPlaneWaves * kWave) void bn_nchw_planes(
    const uint16_t* __restrict__ x, float2* __restrict__ part, NchwMerge mg,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    uint16_t* __restrict__ out, int64_t N, int64_t C, int HW, DivMagic by_hw, int act) {
  constexpr int kVec = (kNchwImages * HWB + kWave - 1) / kWave;  // vectors per lane
  constexpr int kVals = HWB / 8;                                  // plane values per lane
  __shared__ __align__(16) uint16_t stage[kPlaneWaves][kNchwImages * kPlaneChannels * HWB];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x >> 6;
  const int r = lane >> 3;
  const int k = lane & 7;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * kPlaneWaves + w) * kPlaneChannels;
  const bool wave_ok = c0 < C;  // wave-uniform; C % 8 == 0, so all 8 channels exist
  const int64_t s = blockIdx.y;
  const int64_t n0 = s * kNchwImages;
  const int imgs = static_cast<int>(N - n0 < kNchwImages ? N - n0 : kNchwImages);
  const int64_t c = c0 + r;
  u32x4_t* lds = reinterpret_cast<u32x4_t*>(stage[w]);

  // The slice's planes of these 8 channels: image im's block of 8 planes is
  // HW vectors at ((n0 + im) * C + c0) * HW elements; in LDS the blocks sit
  // back to back, vector i of the wave at lds[i].
  // Loads without a branch: slots past the end reload the last vector, and
  // a wave past the last channel block reads the last block (it stores
  // nothing), so all loads are in flight before the first is used.  The
  // epilogue's slice partials, gamma and beta are loaded first, so the merge
  // waits for them alone while x is in flight.
  const int nvec = imgs * HW;
  const int64_t cl = wave_ok ? c0 : C - kPlaneChannels;
  constexpr int kPre = 4;  // slice partials per lane loaded up front
  float2 pre[kPre], first;
  float gc = 0.f, bc = 0.f;
  const float2* pc = nullptr;
  if constexpr (MODE == 1) {
    pc = mg.part + (cl + r) * mg.slices;
    first = pc[0];
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int64_t t = k + 8 * u;
      pre[u] = pc[t < mg.slices ? t : 0];
    }
    gc = gamma[cl + r];
    bc = beta[cl + r];
    __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of x's
  }
  const uint16_t* xb = x + (n0 * C + cl) * static_cast<int64_t>(HW);
  u32x4_t v[kVec];
#pragma unroll
  for (int q = 0; q < kVec; ++q) {
    const int i0 = lane + q * kWave;
    const int i = i0 < nvec ? i0 : nvec - 1;
    const int im = static_cast<int>(div_by(static_cast<uint32_t>(i), by_hw));
    const int64_t off = static_cast<int64_t>(im) * C * HW + static_cast<int64_t>(i - im * HW) * 8;
    v[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(xb + off));
  }

  float mc = 0.f, rc = 0.f;
  if constexpr (MODE == 1) {
    if (wave_ok) {
      const double K = static_cast<double>(first.x);
      double n = 0.0, s1 = 0.0, s2 = 0.0;
      auto add = [&](int64_t t, float2 pv) {
        const int64_t hi = (t + 1) * kNchwImages < N ? (t + 1) * kNchwImages : N;
        const double cnt = static_cast<double>((hi - t * kNchwImages) * HW);
        const double d = static_cast<double>(pv.x) - K;
        n += cnt;
        s1 = __builtin_fma(cnt, d, s1);
        s2 += __builtin_fma(cnt * d, d, static_cast<double>(pv.y));
      };
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        if (k + 8 * u < mg.slices) add(k + 8 * u, pre[u]);
      }
      for (int64_t t = k + 8 * kPre; t < mg.slices; t += 8) add(t, pc[t]);
      n = sum8(n);
      s1 = sum8(s1);
      s2 = sum8(s2);
      const double dm = s1 / n;
      mc = static_cast<float>(K + dm);
      const float var_f = static_cast<float>(std::max(0.0, s2 - s1 * dm) / n);
      rc = 1.0f / __builtin_sqrtf(__fadd_rn(var_f, mg.eps));
      if (s == 0 && k == 0) {
        mg.save_mean[c] = mc;
        mg.save_rstd[c] = rc;
        const float keep = 1.0f - mg.momentum;
        mg.running_mean[c] =
            __fadd_rn(__fmul_rn(mc, mg.momentum), __fmul_rn(mg.running_mean[c], keep));
        mg.running_var[c] = __fadd_rn(__fmul_rn(__fmul_rn(var_f, mg.var_scale), mg.momentum),
                                      __fmul_rn(mg.running_var[c], keep));
      }
    }
  }

#pragma unroll
  for (int q = 0; q < kVec; ++q) {
    const int i = lane + q * kWave;
    if (i < nvec) lds[i] = v[q];
  }
  __syncthreads();
  if (!wave_ok) return;  // wave-uniform, after the only barrier

  // Lane 8r + k's values of plane r of every image: elements k + 8t, read
  // all at once (indices clamped into the plane, values past its end unused).
  const uint16_t* planes = stage[w];
  float val[kNchwImages][kVals];
#pragma unroll
  for (int im = 0; im < kNchwImages; ++im) {
    const int ic = im < imgs ? im : imgs - 1;
    const uint16_t* pl = planes + (ic * kPlaneChannels + r) * HW;
#pragma unroll
    for (int t = 0; t < kVals; ++t) {
      const int j = k + 8 * t;
      val[im][t] = bf16_to_f32(pl[j < HW ? j : HW - 1]);
    }
  }
  if constexpr (MODE == 0) {
    float cnt = 0.f, mean = 0.f, m2 = 0.f;
#pragma unroll
    for (int im = 0; im < kNchwImages; ++im) {
      if (im >= imgs) break;  // wave-uniform
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < kVals; ++t) sum += k + 8 * t < HW ? val[im][t] : 0.f;
      const float mu = sum8(sum) / static_cast<float>(HW);
      float q2 = 0.f;
#pragma unroll
      for (int t = 0; t < kVals; ++t) {
        const float d = val[im][t] - mu;
        q2 = k + 8 * t < HW ? __builtin_fmaf(d, d, q2) : q2;
      }
      chan_merge(cnt, mean, m2, static_cast<float>(HW), mu, sum8(q2));
    }
    if (k == 0) part[c * static_cast<int64_t>(gridDim.y) + s] = make_float2(mean, m2);
  } else {
#pragma unroll
    for (int im = 0; im < kNchwImages; ++im) {
      if (im >= imgs) break;  // wave-uniform
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < kVals; ++t)
        sum += k + 8 * t < HW ? round_bf16(bn_act(val[im][t], mc, rc, gc, bc, act)) : 0.f;
      sum = sum8(sum);
      if (k == 0)
        out[(n0 + im) * C + c] =
            static_cast<uint16_t>(pack_bf16x2(sum / static_cast<float>(HW), 0.f) & 0xffffu);
    }
  }
}

// ---------------------------------------------------------------------------
// NCHW with all of a channel's N x HW values held in registers (C a multiple
// of kChanCh, x and out aligned to a word of kChanCh values, HW <= 64, N * HW
// <= kChanLoads * kChanThreads, ceil(N / kImgStep) * HWB / 8 <=
// kChanMaxVals): one launch, x read once, no workspace.  A workgroup owns
// channels c0 .. c0 + kChanCh - 1; for image n their planes are one
// contiguous run of kChanCh * HW values (HW words), so the workgroup stages
// its N * HW words in LDS ([N][kChanCh][HW] values), all of a thread's
// loads in flight at once.  kChanParts waves share a channel c and split its
// images: wave (ch, part) takes n = kImgStep s + 8 part + r (step s), lane
// 8 r + k the elements k, k + 8, ... of plane (n, c).  From the registers:
//   one pass about shift = x[0, c, 0] (a value of the channel, so the
//     deviations stay of the order of its spread): per lane the sums of
//     d = x - shift and d^2 in fp32, per wave in fp32 (a fixed order), the
//     channel's waves added in order in fp64 through LDS: with n = N HW,
//     mean = shift + S1 / n, M2 = S2 - S1^2 / n (one barrier; the exact
//     two-pass form, mean first and then the squares about it, took a
//     second barrier and 0.5 us more at [128, 1024, 7, 7]);
//   save_mean, save_rstd and the running statistics as the merges elsewhere;
//   out[n, c] = bf16(sum_hw act(bn(x[n, c, hw])) / HW): per step a plane's
//     sum over its 8 lanes (sum8), staged in LDS so that each image's
//     kChanCh outputs leave as one word.
// ---------------------------------------------------------------------------
// Measured at [128, 1024, 7, 7] (ReLU), kernel alone: 4 channels x 4 waves,
// 8-byte words: 11.3 us, 10.6 with the XCD-aware order below (shipped);
// 2 channels x 8 waves, 4-byte words: 16.5 us.  The two-launch planes path
// took 7.5 + 5.8 us there.
constexpr int kChanCh = 4;          // channels per workgroup
typedef u32x2_t chan_word_t;        // kChanCh bf16 values
constexpr int kChanParts = 4;       // waves per channel
constexpr int kChanThreads = kChanCh * kChanParts * kWave;
constexpr int kImgStep = kChanParts * 8;  // images per step of a channel's waves
constexpr int kChanLoads = 8;       // words per thread
constexpr int kChanMaxVals = 32;    // values per lane
constexpr int kChanMaxHw = 64;
constexpr int64_t kChanMaxWords = int64_t{kChanLoads} * kChanThreads;  // N * HW

template <int HWB, int ACT>
__global__ __launch_bounds__(kChanThreads) void bn_nchw_channels(
    const uint16_t* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* __restrict__ running_mean,
    float* __restrict__ running_var, float* __restrict__ save_mean,
    float* __restrict__ save_rstd, uint16_t* __restrict__ out, int N, int C, int HW,
    DivMagic by_hw, float momentum, float eps, float var_scale) {
  constexpr int kT = HWB / 8;                // values per lane per plane
  constexpr int kSteps = kChanMaxVals / kT;  // planes per lane: N <= kImgStep kSteps
  extern __shared__ __align__(16) uint16_t chan_stage[];
  __shared__ double red[2][kChanCh][kChanParts];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int w = t >> 6;
  const int ch = w % kChanCh;
  const int part = w / kChanCh;
  const int r = lane >> 3;
  const int k = lane & 7;
  // XCD-aware order: workgroup ids go round-robin over the 8 XCDs; each XCD
  // takes a contiguous range of channel groups, so the cache lines shared by
  // neighbouring groups' runs are fetched into one L2.
  const int nb = static_cast<int>(gridDim.x);
  const int bid = static_cast<int>(blockIdx.x);
  const int grp = nb % 8 == 0 ? (bid % 8) * (nb / 8) + bid / 8 : bid;
  const int c0 = grp * kChanCh;
  const int c = c0 + ch;
  const int words = N * HW;
  const chan_word_t* xw = reinterpret_cast<const chan_word_t*>(x);
  const float g = gamma[c], b = beta[c];
  chan_word_t v[kChanLoads];
#pragma unroll
  for (int q = 0; q < kChanLoads; ++q) {
    const int i0 = t + q * kChanThreads;
    const int i = i0 < words ? i0 : words - 1;  // in bounds; stored only if i0 < words
    const int n = static_cast<int>(div_by(static_cast<uint32_t>(i), by_hw));
    // Word i - n HW of image n's run, which starts at value (n C + c0) HW,
    // a multiple of kChanCh.
    v[q] = xw[(static_cast<int64_t>(n) * C + c0) * HW / kChanCh + (i - n * HW)];
  }
  chan_word_t* sw = reinterpret_cast<chan_word_t*>(chan_stage);
#pragma unroll
  for (int q = 0; q < kChanLoads; ++q) {
    const int i = t + q * kChanThreads;
    if (i < words) sw[i] = v[q];
  }
  __syncthreads();

  // This lane's values: val[s][u] = x[n_s, c, k + 8u], valid where
  // n_s < N and k + 8u < HW (zero elsewhere).  The LDS reads are
  // unconditional (indices clamped into the staged values), so they all
  // issue before the first is used.
  const uint16_t* pl = chan_stage + ch * HW;
  const int stride = kChanCh * HW;
  float val[kSteps][kT];
  bool img_ok[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int n = kImgStep * s + 8 * part + r;
    img_ok[s] = n < N;
    const uint16_t* p = pl + (img_ok[s] ? n : 0) * stride;
#pragma unroll
    for (int u = 0; u < kT; ++u) {
      const int j = k + 8 * u;
      val[s][u] = bf16_to_f32(p[j < HW ? j : HW - 1]);
    }
  }
#pragma unroll
  for (int s = 0; s < kSteps; ++s)
#pragma unroll
    for (int u = 0; u < kT; ++u) val[s][u] = img_ok[s] && k + 8 * u < HW ? val[s][u] : 0.f;
  const float shift = bf16_to_f32(pl[0]);
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int s = 0; s < kSteps; ++s)
#pragma unroll
    for (int u = 0; u < kT; ++u) {
      const bool ok = img_ok[s] && k + 8 * u < HW;
      const float d = val[s][u] - shift;
      s1 += ok ? d : 0.f;
      s2 = ok ? __builtin_fmaf(d, d, s2) : s2;
    }
  const double w1 = static_cast<double>(wave_sum(s1));
  const double w2 = static_cast<double>(wave_sum(s2));
  if (lane == 0) {
    red[0][ch][part] = w1;
    red[1][ch][part] = w2;
  }
  __syncthreads();
  const double cnt = static_cast<double>(N) * HW;
  double t1 = red[0][ch][0], t2 = red[1][ch][0];
#pragma unroll
  for (int q = 1; q < kChanParts; ++q) {
    t1 += red[0][ch][q];
    t2 += red[1][ch][q];
  }
  const double dmean = t1 / cnt;
  const double mean = static_cast<double>(shift) + dmean;
  const float mf = static_cast<float>(mean);
  const double m2 = t2 - t1 * dmean;
  const float var_f = static_cast<float>(std::max(0.0, m2) / cnt);
  const float rc = 1.0f / __builtin_sqrtf(__fadd_rn(var_f, eps));
  if (part == 0 && lane == 0) {
    save_mean[c] = mf;
    save_rstd[c] = rc;
    const float keep = 1.0f - momentum;
    running_mean[c] = __fadd_rn(__fmul_rn(mf, momentum), __fmul_rn(running_mean[c], keep));
    running_var[c] = __fadd_rn(__fmul_rn(__fmul_rn(var_f, var_scale), momentum),
                               __fmul_rn(running_var[c], keep));
  }
  // The staged x is no longer read (every wave passed the barriers above
  // after its last read of it): the outputs go there, [N][kChanCh].
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    if (kImgStep * s >= N) break;  // wave-uniform
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < kT; ++u)
      sum += k + 8 * u < HW ? round_bf16(bn_act(val[s][u], mf, rc, g, b, ACT)) : 0.f;
    sum = sum8(sum);
    const int n = kImgStep * s + 8 * part + r;
    if (k == 0 && img_ok[s])
      chan_stage[n * kChanCh + ch] =
          static_cast<uint16_t>(pack_bf16x2(sum / static_cast<float>(HW), 0.f) & 0xffffu);
  }
  __syncthreads();
  chan_word_t* ow = reinterpret_cast<chan_word_t*>(out);
  for (int n = t; n < N; n += kChanThreads)
    ow[(static_cast<int64_t>(n) * C + c0) / kChanCh] = sw[n];
}

// ---------------------------------------------------------------------------
// Per-channel merge.  The workspace is channel-major: part[c * S + s] is
// slice s of channel c, which holds (min(units, (s+1)*per) - s*per) * mult
// values with mean m_s and M2_s.  In fp64, about the shift K = m_0:
// S1 = sum n_s (m_s - K), S2 = sum M2_s + n_s (m_s - K)^2 -- a plain sum, no
// divisions.  A workgroup of kFinalThreads threads per channel: thread t
// adds slices t, t + kFinalThreads, ... (the first kFinalLoads of them
// loaded at once), a butterfly adds the lanes of each wave, and thread 0
// adds the waves in order.  mean = K + S1 / N, M2 = S2 - S1^2 / N.
// ---------------------------------------------------------------------------
constexpr int kFinalThreads = 256;
constexpr int kFinalLoads = 4;

__global__ __launch_bounds__(kFinalThreads) void bn_finalize(
    const float2* __restrict__ part, int64_t slices, int64_t units, int64_t per, int64_t mult,
    float* __restrict__ running_mean, float* __restrict__ running_var,
    float* __restrict__ save_mean, float* __restrict__ save_rstd, float momentum, float eps,
    float var_scale) {
  __shared__ double wsum[kFinalThreads / kWave][3];
  const int64_t c = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const float2* pc = part + c * slices;
  const double K = static_cast<double>(pc[0].x);
  double n = 0.0, s1 = 0.0, s2 = 0.0;
  auto add = [&](int64_t s, float2 p) {
    const double cnt =
        s < slices
            ? static_cast<double>((std::min<int64_t>(units, (s + 1) * per) - s * per) * mult)
            : 0.0;
    const double d = static_cast<double>(p.x) - K;
    n += cnt;
    s1 = __builtin_fma(cnt, d, s1);
    s2 += cnt > 0.0 ? __builtin_fma(cnt * d, d, static_cast<double>(p.y)) : 0.0;
  };
  float2 v[kFinalLoads];
#pragma unroll
  for (int k = 0; k < kFinalLoads; ++k) {
    const int64_t s = t + static_cast<int64_t>(k) * kFinalThreads;
    v[k] = pc[s < slices ? s : 0];
  }
#pragma unroll
  for (int k = 0; k < kFinalLoads; ++k) add(t + static_cast<int64_t>(k) * kFinalThreads, v[k]);
  for (int64_t s = t + int64_t{kFinalLoads} * kFinalThreads; s < slices; s += kFinalThreads)
    add(s, pc[s]);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    // (lower lane) + (upper lane) in both lanes: the same rounding everywhere
    const double n2 = __shfl_xor(n, off), a2 = __shfl_xor(s1, off), b2 = __shfl_xor(s2, off);
    const bool upper = (lane & off) != 0;
    n = upper ? n2 + n : n + n2;
    s1 = upper ? a2 + s1 : s1 + a2;
    s2 = upper ? b2 + s2 : s2 + b2;
  }
  if (lane == 0) {
    wsum[t / kWave][0] = n;
    wsum[t / kWave][1] = s1;
    wsum[t / kWave][2] = s2;
  }
  __syncthreads();
  if (t != 0) return;
  for (int w = 1; w < kFinalThreads / kWave; ++w) {
    n += wsum[w][0];
    s1 += wsum[w][1];
    s2 += wsum[w][2];
  }
  const double dm = s1 / n;
  const float mean_f = static_cast<float>(K + dm);
  const float var_f = static_cast<float>(std::max(0.0, s2 - s1 * dm) / n);
  save_mean[c] = mean_f;
  save_rstd[c] = 1.0f / __builtin_sqrtf(__fadd_rn(var_f, eps));
  const float keep = 1.0f - momentum;
  running_mean[c] = __fadd_rn(__fmul_rn(mean_f, momentum), __fmul_rn(running_mean[c], keep));
  running_var[c] = __fadd_rn(__fmul_rn(__fmul_rn(var_f, var_scale), momentum),
                             __fmul_rn(running_var[c], keep));
}

int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Channels-last plan: threads per workgroup (0: scalar kernels), rows per
// slice and slice count.  Slices of a multiple of 512 rows, at most about
// 512 of them; the slicing does not depend on the kernel choice, so the
// workspace size is a function of the shape alone.  The workspace traffic
// (8 B per channel per slice) stays under 1 % of x for the corpus shapes.
// Measured on MI355X (statistics kernel, [128, 240, 28, 28] / [128, 96,
// 112, 112]): 512-row slices, at most 512 of them, 8 non-temporal loads in
// flight per thread: 15.2 / 49.9 us; at most 1024 / 256 / 128 slices:
// 61.8 / 53.6 / 84.8 us on the second shape; 256-row slices, 4 or 16 loads,
// or cached loads: 21-27 / 55-64 us.  Whole call (three launches, graph
// loop): 44.0 / 160.2 us as planned; 128- or 64-row slices with up to 1024
// or 2048 of them 71-100 / 167-184 us; 2 or 1 rows per thread in the
// epilogue instead of kApplyUnroll = 4: 44.1-51.2 / 168.6-203.5 us.  With
// the SiLU fast form, one call after a 1 GiB cache flush (the runner's
// protocol), [128, 240, 28, 28] / [128, 96, 112, 112]: 47.2 / 161-163 us
// with 960-thread workgroups and non-temporal loads; 42.5 / 162.5 with 480
// threads (G * R above); 38.4 / 161.5 with 480 threads, cached loads and
// the reversed epilogue (shipped); 256-row slices on top: 40.7 / 162.6.
struct NhwcPlan {
  int threads = 0;
  int64_t slice_len = 0;
  int64_t slices = 0;
};

constexpr int64_t kNhwcSliceStep = 512;
constexpr int64_t kNhwcMaxSlices = 512;

NhwcPlan nhwc_plan(int64_t M, int64_t C, bool vec_ok) {
  NhwcPlan plan;
  if (M <= 0 || C <= 0) return plan;
  if (vec_ok && C % 8 == 0 && C / 8 <= kMaxThreads) {
    const int64_t G = C / 8;
    const int64_t lcm = G / gcd64(G, kWave) * kWave;
    if (lcm <= 512) {
      plan.threads = static_cast<int>(lcm * (512 / lcm));
    } else {
      // Whole waves would take lcm threads (960 for C = 240): one such
      // workgroup per CU at the kernels' register use.  G * R threads with
      // a partial last wave fit two or three per CU instead.
      int64_t R = 1;
      while (G * R * 2 <= 512) R *= 2;
      plan.threads = static_cast<int>(G * R);
    }
  }
  const int64_t want = (M + kNhwcMaxSlices - 1) / kNhwcMaxSlices;
  plan.slice_len = (want + kNhwcSliceStep - 1) / kNhwcSliceStep * kNhwcSliceStep;
  plan.slices = (M + plan.slice_len - 1) / plan.slice_len;
  return plan;
}

int64_t nchw_slices(int64_t n) { return (n + kNchwImages - 1) / kNchwImages; }

}  // namespace
}  // namespace hipo

extern "C" size_t hipo_batchnorm_nhwc_workspace_bytes(int64_t n, int64_t h, int64_t w,
                                                     int64_t c) {
  if (n <= 0 || h <= 0 || w <= 0 || c <= 0) return 0;
  const hipo::NhwcPlan plan = hipo::nhwc_plan(n * h * w, c, true);
  return static_cast<size_t>(plan.slices * c) * sizeof(float2);
}

extern "C" int hipo_batchnorm_nhwc_act_pad_bf16(
    const uint16_t* x, const float* gamma, const float* beta, float* running_mean,
    float* running_var, float* save_mean, float* save_rstd, uint16_t* out, int64_t n, int64_t h,
    int64_t w, int64_t c, int64_t pad_bottom, int64_t pad_right, float momentum, float eps,
    float var_scale, int act, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  const char* what = "batchnorm_nhwc_act_pad_bf16";
  HIPO_REQUIRE(n >= 0 && h >= 0 && w >= 0 && c >= 0 && pad_bottom >= 0 && pad_right >= 0,
               "%s: negative size", what);
  HIPO_REQUIRE(act >= kActNone && act <= kActSilu, "%s: act must be 0, 1 or 2", what);
  if (c == 0) return 0;
  HIPO_REQUIRE(n > 0 && h > 0 && w > 0, "%s: empty reduction (n * h * w == 0)", what);
  HIPO_REQUIRE(x && gamma && beta && running_mean && running_var && save_mean && save_rstd && out,
               "%s: null pointer", what);
  const int64_t M = n * h * w;
  const int64_t Ho = h + pad_bottom, Wo = w + pad_right;
  const int64_t rows_out = n * Ho * Wo;
  const bool vec_ok = aligned16(x) && aligned16(out) && rows_out < (int64_t{1} << 31) &&
                      M < (int64_t{1} << 31);
  const NhwcPlan plan = nhwc_plan(M, c, vec_ok);
  const size_t need = static_cast<size_t>(plan.slices * c) * sizeof(float2);
  HIPO_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
               "%s: workspace of %zu bytes (16-byte aligned), need %zu", what, workspace_bytes,
               need);
  HIPO_REQUIRE(plan.slices <= 65535 || plan.threads > 0, "%s: too many rows", what);
  float2* part = static_cast<float2*>(workspace);
  if (plan.threads > 0) {
    const int G = static_cast<int>(c / 8);
    const int R = plan.threads / G;
    HIPO_REQUIRE((R & (R - 1)) == 0, "%s: rows per instruction %d not a power of two", what, R);
    const size_t lds = R > 1 ? static_cast<size_t>(plan.threads / 2) * 16 * sizeof(float) : 0;
    bn_nhwc_partial<<<dim3(static_cast<unsigned>(plan.slices)), dim3(plan.threads), lds,
                      stream>>>(x, part, M, c, G, plan.slice_len);
  } else {
    bn_nhwc_partial_scalar<<<dim3(static_cast<unsigned>((c + 255) / 256),
                                  static_cast<unsigned>(plan.slices)),
                             dim3(256), 0, stream>>>(x, part, M, c, plan.slice_len);
  }
  bn_finalize<<<dim3(static_cast<unsigned>(c)), dim3(kFinalThreads), 0, stream>>>(
      part, plan.slices, M, plan.slice_len, 1, running_mean, running_var, save_mean, save_rstd,
      momentum, eps, var_scale);
  if (plan.threads > 0) {
    const int G = static_cast<int>(c / 8);
    const int64_t rows_per_block = static_cast<int64_t>(plan.threads / G) * kApplyUnroll;
    const int64_t blocks = (rows_out + rows_per_block - 1) / rows_per_block;
    auto kernel = act == kActSilu   ? bn_nhwc_apply_pad<kActSilu>
                  : act == kActRelu ? bn_nhwc_apply_pad<kActRelu>
                                    : bn_nhwc_apply_pad<kActNone>;
    kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(plan.threads), 0, stream>>>(
        x, save_mean, save_rstd, gamma, beta, out, static_cast<uint32_t>(rows_out),
        static_cast<uint32_t>(h), static_cast<uint32_t>(w), static_cast<uint32_t>(Ho),
        static_cast<uint32_t>(Wo), div_magic(static_cast<uint32_t>(Ho * Wo)),
        div_magic(static_cast<uint32_t>(Wo)), G);
  } else {
    const int64_t total = rows_out * c;
    HIPO_REQUIRE((total + 255) / 256 <= 0x7fffffff, "%s: too large", what);
    bn_nhwc_apply_pad_scalar<<<dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                               stream>>>(x, save_mean, save_rstd, gamma, beta, out, total, h, w,
                                         Ho, Wo, c, act);
  }
  return check_launch(what);
}

extern "C" size_t hipo_batchnorm_nchw_mean_workspace_bytes(int64_t n, int64_t c, int64_t hw) {
  if (n <= 0 || c <= 0 || hw <= 0) return 0;
  return static_cast<size_t>(hipo::nchw_slices(n) * c) * sizeof(float2);
}

extern "C" int hipo_batchnorm_nchw_act_mean_bf16(
    const uint16_t* x, const float* gamma, const float* beta, float* running_mean,
    float* running_var, float* save_mean, float* save_rstd, uint16_t* out, int64_t n, int64_t c,
    int64_t hw, float momentum, float eps, float var_scale, int act, void* workspace,
    size_t workspace_bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  const char* what = "batchnorm_nchw_act_mean_bf16";
  HIPO_REQUIRE(n >= 0 && c >= 0 && hw >= 0, "%s: negative size", what);
  HIPO_REQUIRE(act >= kActNone && act <= kActSilu, "%s: act must be 0, 1 or 2", what);
  if (c == 0) return 0;
  HIPO_REQUIRE(n > 0 && hw > 0, "%s: empty reduction (n * hw == 0)", what);
  HIPO_REQUIRE(x && gamma && beta && running_mean && running_var && save_mean && save_rstd && out,
               "%s: null pointer", what);
  const int64_t slices = nchw_slices(n);
  const size_t need = static_cast<size_t>(slices * c) * sizeof(float2);
  HIPO_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
               "%s: workspace of %zu bytes (16-byte aligned), need %zu", what, workspace_bytes,
               need);
  HIPO_REQUIRE(slices <= 65535, "%s: too many images", what);
  const bool word_aligned = reinterpret_cast<uintptr_t>(x) % sizeof(chan_word_t) == 0 &&
                            reinterpret_cast<uintptr_t>(out) % sizeof(chan_word_t) == 0;
  if (c % kChanCh == 0 && word_aligned && hw <= kChanMaxHw && n * hw <= kChanMaxWords) {
    const int hwb = hw <= 8 ? 8 : hw <= 16 ? 16 : hw <= 32 ? 32 : 64;
    if ((n + kImgStep - 1) / kImgStep * (hwb / 8) <= kChanMaxVals) {
      const int ni = static_cast<int>(n), ci = static_cast<int>(c), hi = static_cast<int>(hw);
      const DivMagic by_hw = div_magic(static_cast<uint32_t>(hw));
      const size_t lds = static_cast<size_t>(n * hw) * sizeof(chan_word_t);
      const dim3 grid(static_cast<unsigned>(c / kChanCh));
      const dim3 block(kChanThreads);
#define HIPO_CHANNELS(B_)                                                                        \
  do {                                                                                           \
    auto kernel = act == kActSilu   ? bn_nchw_channels<B_, kActSilu>                             \
                  : act == kActRelu ? bn_nchw_channels<B_, kActRelu>                             \
                                    : bn_nchw_channels<B_, kActNone>;                            \
    kernel<<<grid, block, lds, stream>>>(x, gamma, beta, running_mean, running_var, save_mean,   \
                                         save_rstd, out, ni, ci, hi, by_hw, momentum, eps,       \
                                         var_scale);                                             \
  } while (0)
      if (hwb == 8) {
        HIPO_CHANNELS(8);
      } else if (hwb == 16) {
        HIPO_CHANNELS(16);
      } else if (hwb == 32) {
        HIPO_CHANNELS(32);
      } else {
        HIPO_CHANNELS(64);
      }
#undef HIPO_CHANNELS
      return check_launch(what);
    }
  }
  float2* part = static_cast<float2*>(workspace);
  const NchwMerge none{};
  const NchwMerge mg{part, slices, running_mean, running_var, save_mean, save_rstd,
                     momentum, eps, var_scale};
  if (c % kPlaneChannels == 0 && hw <= kPlanesMaxHw && aligned16(x)) {
    const int64_t cb = (c + kPlaneWaves * kPlaneChannels - 1) / (kPlaneWaves * kPlaneChannels);
    const dim3 grid(static_cast<unsigned>(cb), static_cast<unsigned>(slices));
    const dim3 block(kPlaneWaves * kWave);
    const int h = static_cast<int>(hw);
    const DivMagic by_hw = div_magic(static_cast<uint32_t>(hw));
#define HIPO_PLANES(B_)                                                                      \
  do {                                                                                       \
    bn_nchw_planes<0, B_><<<grid, block, 0, stream>>>(x, part, none, nullptr, nullptr,        \
                                                      nullptr, n, c, h, by_hw, act);         \
    bn_nchw_planes<1, B_><<<grid, block, 0, stream>>>(x, nullptr, mg, gamma, beta, out, n, c, \
                                                      h, by_hw, act);                        \
  } while (0)
    if (hw <= 8) {
      HIPO_PLANES(8);
    } else if (hw <= 16) {
      HIPO_PLANES(16);
    } else if (hw <= 32) {
      HIPO_PLANES(32);
    } else if (hw <= 64) {
      HIPO_PLANES(64);
    } else {
      HIPO_PLANES(128);
    }
#undef HIPO_PLANES
  } else {
    const dim3 grid(static_cast<unsigned>((c + kNchwChannels - 1) / kNchwChannels),
                    static_cast<unsigned>(slices));
    const dim3 block(kNchwImages * kWave);
    bn_nchw_small_hw<0><<<grid, block, 0, stream>>>(x, part, none, nullptr, nullptr, nullptr,
                                                    n, c, hw, act);
    bn_nchw_small_hw<1><<<grid, block, 0, stream>>>(x, nullptr, mg, gamma, beta, out, n, c, hw,
                                                    act);
  }
  return check_launch(what);
}
