// BatchNorm training forward, fp32 NCHW: per-channel statistics over
// (N, H, W), normalisation + affine (+ ReLU), running-stat update.
//
// Entry point.  Channels of at most 16384 values take one launch with a
// workgroup per channel that holds its channel in registers
// (bn_channel_small).  Larger channels take the single-pass persistent
// kernel (batchnorm_fused.hip) wherever it applies, and the split-K path
// below otherwise (HW not a multiple of 4, unaligned pointers, very large
// tensors, more than 64 workgroups per channel or 64 rounds).
//
// Split-K structure (two launches on the caller's stream):
//   1. bn_partial_stats: grid (S, C).  Workgroup (s, c) reduces the planes
//      n in [s*N/S, (s+1)*N/S) of channel c to a Welford triple
//      (count, mean, M2) and writes it to the workspace.  Inside the
//      workgroup each thread reduces its slice of every plane exactly
//      (two-pass over registers) and merges it into a running triple with
//      Chan's formula; threads then merge across the wave with DPP and
//      across waves through LDS.
//   2. bn_normalize: grid (S, C).  Every workgroup of channel c merges the S
//      triples of that channel (Chan, fp64, fixed order), derives
//      mean / invstd, and writes y = relu?(x * alpha + beta') for its planes
//      with alpha = invstd * gamma, beta' = beta - mean * alpha.  Workgroup
//      (0, c) also writes save_mean / save_invstd and updates the running
//      statistics (unbiased variance, count / (count - 1)).
// This path reads x twice (once per launch).
#include <mutex>
#include <type_traits>

#include "welford.h"

namespace hipo {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

// max(v, 0) that keeps NaN (torch.relu propagates NaN; fmaxf would not).
__device__ __forceinline__ float relu_f32(float v) { return v < 0.f ? 0.f : v; }

// Exact statistics of up to 4*U values held by one thread, merged into acc.
template <int U>
__device__ __forceinline__ void absorb(Welford& acc, const float4 (&v)[U],
                                       const bool (&ok)[U]) {
  float cnt = 0.f, s = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (ok[u]) {
      cnt += 4.f;
      s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
  }
  if (cnt == 0.f) return;
  const float m = s / cnt;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (ok[u]) {
      const float a = v[u].x - m, b = v[u].y - m, c = v[u].z - m, d = v[u].w - m;
      q += (a * a + b * b) + (c * c + d * d);
    }
  }
  acc = welford_merge(acc, Welford{cnt, m, q});
}

// The same for up to U single values.
template <int U>
__device__ __forceinline__ void absorb(Welford& acc, const float (&v)[U], const bool (&ok)[U]) {
  float cnt = 0.f, s = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (ok[u]) {
      cnt += 1.f;
      s += v[u];
    }
  }
  if (cnt == 0.f) return;
  const float m = s / cnt;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (ok[u]) q += (v[u] - m) * (v[u] - m);
  }
  acc = welford_merge(acc, Welford{cnt, m, q});
}

// Planes handled by split s of S over N planes.
__device__ __forceinline__ void split_range(int64_t N, int64_t S, int64_t s,
                                            int64_t& n0, int64_t& n1) {
  n0 = (N * s) / S;
  n1 = (N * (s + 1)) / S;
}

// Merge the threads' triples: DPP across the wave, LDS across the waves.
// Every thread returns the workgroup's total.
__device__ __forceinline__ Welford block_welford(Welford acc) {
  acc = wave_welford(acc);
  __shared__ Welford part[kWavesPerBlock];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & (kWave - 1)) == 0) part[wave] = acc;
  __syncthreads();
  return welford_merge(welford_merge(part[0], part[1]), welford_merge(part[2], part[3]));
}

// Welford triple of planes [n0, n1) of channel c over the workgroup: each
// thread reduces its slice of every plane exactly (two-pass over registers)
// and merges it into a running triple with Chan's formula; the wave merges
// with DPP and the waves through LDS.  Thread 0 returns the total.
template <bool VEC>
__device__ Welford planes_welford(const float* __restrict__ x, int64_t n0, int64_t n1,
                                  int64_t C, int64_t HW, int64_t c) {
  Welford acc{0.f, 0.f, 0.f};
  if constexpr (VEC) {
    constexpr int U = 4;
    const int64_t hw4 = HW / 4;
    for (int64_t n = n0; n < n1; ++n) {
      const float4* plane = reinterpret_cast<const float4*>(x + (n * C + c) * HW);
      for (int64_t base = 0; base < hw4; base += kThreads * U) {
        float4 v[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t i = base + u * kThreads + threadIdx.x;
          ok[u] = i < hw4;
          v[u] = ok[u] ? plane[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        absorb<U>(acc, v, ok);
      }
    }
  } else {
    for (int64_t n = n0; n < n1; ++n) {
      const float* plane = x + (n * C + c) * HW;
      for (int64_t i = threadIdx.x; i < HW; i += kThreads) {
        acc = welford_merge(acc, Welford{1.f, plane[i], 0.f});
      }
    }
  }
  return block_welford(acc);
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void bn_partial_stats(
    const float* __restrict__ x, float* __restrict__ ws, int64_t N, int64_t C,
    int64_t HW, int64_t S) {
  const int64_t s = blockIdx.x;
  const int64_t c = blockIdx.y;
  int64_t n0, n1;
  split_range(N, S, s, n0, n1);
  const Welford t = planes_welford<VEC>(x, n0, n1, C, HW, c);
  if (threadIdx.x == 0) {
    float* dst = ws + (c * S + s) * 3;
    dst[0] = t.n;
    dst[1] = t.mean;
    dst[2] = t.m2;
  }
}

// Merge the S partial triples of channel c in fp64, fixed order.
__device__ void channel_stats(const float* __restrict__ ws, int64_t c,
                              int64_t S, double& mean, double& m2,
                              double& count) {
  double n = 0.0, mu = 0.0, q = 0.0;
  for (int64_t s = 0; s < S; ++s) {
    const float* p = ws + (c * S + s) * 3;
    const double nb = p[0], mb = p[1], qb = p[2];
    const double nn = n + nb;
    if (nn == 0.0) continue;
    const double d = mb - mu;
    mu += d * (nb / nn);
    q += qb + d * d * n * (nb / nn);
    n = nn;
  }
  mean = mu;
  m2 = q;
  count = n;
}

// mean / invstd from the merged (mean, M2, count) of channel c -> the
// affine coefficients (alpha = invstd * gamma, shift = beta - mean * alpha)
// in coef[0..1]; with write_stats, save_mean / save_invstd and the running
// statistics (unbiased variance, count / (count - 1)).
// channel_coefs with gamma[c], beta[c] and the running statistics already
// loaded (g, b, rm, rv).
__device__ void channel_coefs_of(double mean, double m2, double count, int64_t c, float g,
                                 float b, float rm, float rv, float* __restrict__ running_mean,
                                 float* __restrict__ running_var, float* __restrict__ save_mean,
                                 float* __restrict__ save_invstd, float momentum, float eps,
                                 bool write_stats, float* coef) {
  const float meanf = static_cast<float>(mean);
  const float var = static_cast<float>(m2 / count);
  const float invstd = 1.0f / __builtin_sqrtf(var + eps);
  const float alpha = invstd * g;
  coef[0] = alpha;
  coef[1] = b - meanf * alpha;
  if (write_stats) {
    save_mean[c] = meanf;
    save_invstd[c] = invstd;
    const double unbiased = count > 1.0 ? m2 / (count - 1.0) : __builtin_nan("");
    const double mom = momentum;
    running_mean[c] = static_cast<float>(mom * mean + (1.0 - mom) * rm);
    running_var[c] = static_cast<float>(mom * unbiased + (1.0 - mom) * rv);
  }
}

__device__ void channel_coefs(double mean, double m2, double count, int64_t c,
                              const float* __restrict__ gamma, const float* __restrict__ beta,
                              float* __restrict__ running_mean, float* __restrict__ running_var,
                              float* __restrict__ save_mean, float* __restrict__ save_invstd,
                              float momentum, float eps, bool write_stats, float* coef) {
  channel_coefs_of(mean, m2, count, c, gamma[c], beta[c], write_stats ? running_mean[c] : 0.f,
                   write_stats ? running_var[c] : 0.f, running_mean, running_var, save_mean,
                   save_invstd, momentum, eps, write_stats, coef);
}

// y = relu?(x * alpha + shift) over planes [n0, n1) of channel c.
template <bool VEC>
__device__ void normalize_planes(const float* __restrict__ x, float* __restrict__ y,
                                 int64_t n0, int64_t n1, int64_t C, int64_t HW, int64_t c,
                                 float alpha, float shift, int relu) {
  for (int64_t n = n0; n < n1; ++n) {
    const int64_t off = (n * C + c) * HW;
    if (VEC) {
      const float4* src = reinterpret_cast<const float4*>(x + off);
      float4* dst = reinterpret_cast<float4*>(y + off);
      for (int64_t i = threadIdx.x; i < HW / 4; i += kThreads) {
        float4 v = src[i];
        v.x = __builtin_fmaf(v.x, alpha, shift);
        v.y = __builtin_fmaf(v.y, alpha, shift);
        v.z = __builtin_fmaf(v.z, alpha, shift);
        v.w = __builtin_fmaf(v.w, alpha, shift);
        if (relu) {
          v.x = relu_f32(v.x);
          v.y = relu_f32(v.y);
          v.z = relu_f32(v.z);
          v.w = relu_f32(v.w);
        }
        dst[i] = v;
      }
    } else {
      for (int64_t i = threadIdx.x; i < HW; i += kThreads) {
        float v = __builtin_fmaf(x[off + i], alpha, shift);
        if (relu) v = relu_f32(v);
        y[off + i] = v;
      }
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void bn_normalize(
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* __restrict__ running_mean,
    float* __restrict__ running_var, float* __restrict__ y,
    float* __restrict__ save_mean, float* __restrict__ save_invstd,
    const float* __restrict__ ws, int64_t N, int64_t C, int64_t HW, int64_t S,
    float momentum, float eps, int relu) {
  const int64_t s = blockIdx.x;
  const int64_t c = blockIdx.y;
  __shared__ float coef[2];
  if (threadIdx.x == 0) {
    double mean, m2, count;
    channel_stats(ws, c, S, mean, m2, count);
    channel_coefs(mean, m2, count, c, gamma, beta, running_mean, running_var, save_mean,
                  save_invstd, momentum, eps, s == 0, coef);
  }
  __syncthreads();
  int64_t n0, n1;
  split_range(N, S, s, n0, n1);
  normalize_planes<VEC>(x, y, n0, n1, C, HW, c, coef[0], coef[1], relu);
}

// Small channels (N * HW <= kSmallChannel values): one launch, a workgroup
// per channel holding the channel in registers -- U float4 (or U single
// values when HW % 4 != 0 or x, y are unaligned) per thread, every load in
// flight at once, with gamma, beta and the running statistics loaded beside
// them.  Exact per-thread statistics (two-pass over the registers), Chan
// merges across the wave and the workgroup, fp64 coefficients (the split-K
// path's arithmetic with one split), then y written from the registers: x
// is read once, and the chain from launch to the last store holds a single
// memory round trip for the data.  At ragged points such as [3, 5, 7, 7]
// or [4, 24, 10, 10] that chain, not the bytes, is the time (the
// single-pass kernel adds an epoch read and a slab exchange to it).
constexpr int64_t kSmallChannel = 16384;

struct SmallGeom {
  int total;      // float4 (VEC) or values per channel
  int per_plane;  // HW / 4 (VEC) or HW
  DivMagic by_plane;
};

template <bool VEC, int U>
__global__ __launch_bounds__(kThreads) void bn_channel_small(
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* __restrict__ running_mean,
    float* __restrict__ running_var, float* __restrict__ y,
    float* __restrict__ save_mean, float* __restrict__ save_invstd, SmallGeom g, int64_t C,
    float momentum, float eps, int relu) {
  using Elem = std::conditional_t<VEC, float4, float>;
  const int64_t c = blockIdx.x;
  float pg = 0.f, pb = 0.f, prm = 0.f, prv = 0.f;
  if (threadIdx.x == 0) {
    pg = gamma[c];
    pb = beta[c];
    prm = running_mean[c];
    prv = running_var[c];
  }
  // Element i of the channel: plane i / per_plane, offset i % per_plane.
  auto offset = [&](int i) {
    const uint32_t n = div_by(static_cast<uint32_t>(i), g.by_plane);
    return (static_cast<int64_t>(n) * C + c) * g.per_plane +
           (i - static_cast<int>(n) * g.per_plane);
  };
  const Elem* xs = reinterpret_cast<const Elem*>(x);
  Elem v[U];
  bool ok[U];
  // Unconditional loads (threads past the channel's end re-read its last
  // element and store nothing), so all of them are in flight together.
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = static_cast<int>(threadIdx.x) + u * kThreads;
    ok[u] = i < g.total;
    v[u] = xs[offset(ok[u] ? i : g.total - 1)];
  }
  Welford acc{0.f, 0.f, 0.f};
  absorb<U>(acc, v, ok);
  const Welford t = block_welford(acc);
  __shared__ float coef[2];
  if (threadIdx.x == 0)
    channel_coefs_of(static_cast<double>(t.mean), static_cast<double>(t.m2),
                     static_cast<double>(t.n), c, pg, pb, prm, prv, running_mean, running_var,
                     save_mean, save_invstd, momentum, eps, true, coef);
  __syncthreads();
  const float alpha = coef[0], shift = coef[1];
  Elem* ys = reinterpret_cast<Elem*>(y);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!ok[u]) continue;
    Elem o = v[u];
    if constexpr (VEC) {
      o.x = __builtin_fmaf(o.x, alpha, shift);
      o.y = __builtin_fmaf(o.y, alpha, shift);
      o.z = __builtin_fmaf(o.z, alpha, shift);
      o.w = __builtin_fmaf(o.w, alpha, shift);
      if (relu) {
        o.x = relu_f32(o.x);
        o.y = relu_f32(o.y);
        o.z = relu_f32(o.z);
        o.w = relu_f32(o.w);
      }
    } else {
      o = __builtin_fmaf(o, alpha, shift);
      if (relu) o = relu_f32(o);
    }
    ys[offset(static_cast<int>(threadIdx.x) + u * kThreads)] = o;
  }
}

template <bool VEC, int U>
void launch_small(const float* x, const float* gamma, const float* beta, float* running_mean,
                  float* running_var, float* y, float* save_mean, float* save_invstd,
                  const SmallGeom& g, int64_t c, float momentum, float eps, int relu,
                  hipStream_t stream) {
  bn_channel_small<VEC, U><<<dim3(static_cast<unsigned>(c)), dim3(kThreads), 0, stream>>>(
      x, gamma, beta, running_mean, running_var, y, save_mean, save_invstd, g, c, momentum,
      eps, relu);
}

// U = the smallest instantiated count covering the channel.
int small_launch(const float* x, const float* gamma, const float* beta, float* running_mean,
                 float* running_var, float* y, float* save_mean, float* save_invstd, int64_t n,
                 int64_t c, int64_t hw, float momentum, float eps, int relu,
                 hipStream_t stream) {
  const bool vec = hw % 4 == 0 && aligned16(x) && aligned16(y);
  SmallGeom g;
  g.per_plane = static_cast<int>(vec ? hw / 4 : hw);
  g.total = static_cast<int>(n) * g.per_plane;
  g.by_plane = div_magic(static_cast<uint32_t>(g.per_plane));
  const int per_thread = (g.total + kThreads - 1) / kThreads;
#define HIPO_BN_SMALL(V, U)                                                              \
  launch_small<V, U>(x, gamma, beta, running_mean, running_var, y, save_mean, save_invstd, \
                     g, c, momentum, eps, relu, stream)
  if (vec) {
    if (per_thread <= 1) HIPO_BN_SMALL(true, 1);
    else if (per_thread <= 2) HIPO_BN_SMALL(true, 2);
    else if (per_thread <= 4) HIPO_BN_SMALL(true, 4);
    else if (per_thread <= 8) HIPO_BN_SMALL(true, 8);
    else HIPO_BN_SMALL(true, 16);
  } else {
    if (per_thread <= 1) HIPO_BN_SMALL(false, 1);
    else if (per_thread <= 4) HIPO_BN_SMALL(false, 4);
    else if (per_thread <= 16) HIPO_BN_SMALL(false, 16);
    else HIPO_BN_SMALL(false, 64);
  }
#undef HIPO_BN_SMALL
  return check_launch("batchnorm_train_fwd_f32 (small channels)");
}

// Number of plane splits per channel for the split-K launches.
int64_t num_splits(int64_t n, int64_t c) {
  const int64_t target_blocks = 4096;
  int64_t s = (target_blocks + c - 1) / c;
  if (s > n) s = n;
  if (s < 1) s = 1;
  return s;
}

}  // namespace
}  // namespace hipo

extern "C" size_t hipo_batchnorm_workspace_bytes(int64_t n, int64_t c,
                                                 int64_t hw) {
  if (n <= 0 || c <= 0 || hw <= 0) return 0;
  const int64_t s = hipo::num_splits(n, c);
  return hipo::kBnCtlBytes + hipo::bn_fused_slot_bytes(n, c, hw) +
         static_cast<size_t>(c * s * 3) * sizeof(float);
}

extern "C" int hipo_batchnorm_train_fwd_f32(
    const float* x, const float* gamma, const float* beta, float* running_mean,
    float* running_var, float* y, float* save_mean, float* save_invstd,
    int64_t n, int64_t c, int64_t hw, float momentum, float eps, int relu,
    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n > 0 && c > 0 && hw > 0, "batchnorm: sizes must be positive");
  HIPO_REQUIRE(x && gamma && beta && running_mean && running_var && y &&
                   save_mean && save_invstd && workspace,
               "batchnorm: null pointer");
  const size_t need = hipo_batchnorm_workspace_bytes(n, c, hw);
  HIPO_REQUIRE(workspace_bytes >= need,
               "batchnorm: workspace %zu bytes < required %zu", workspace_bytes,
               need);
  HIPO_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 8 == 0,
               "batchnorm: workspace must be 8-byte aligned");
  if (n * hw <= kSmallChannel && c <= 0x7fffffff)
    return small_launch(x, gamma, beta, running_mean, running_var, y, save_mean, save_invstd,
                        n, c, hw, momentum, eps, relu, stream);
  const int fused = bn_fused_launch(x, gamma, beta, running_mean, running_var, y,
                                    save_mean, save_invstd, n, c, hw, momentum,
                                    eps, relu, workspace, stream);
  if (fused >= 0) return fused;

  const bool vec = hw % 4 == 0 && aligned16(x) && aligned16(y);

  HIPO_REQUIRE(c <= 65535, "batchnorm: too many channels");
  const int64_t S = num_splits(n, c);
  const dim3 grid(static_cast<unsigned>(S), static_cast<unsigned>(c));
  float* ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kBnCtlBytes +
                                       bn_fused_slot_bytes(n, c, hw));
  if (vec) {
    bn_partial_stats<true><<<grid, dim3(kThreads), 0, stream>>>(x, ws, n, c, hw, S);
  } else {
    bn_partial_stats<false><<<grid, dim3(kThreads), 0, stream>>>(x, ws, n, c, hw, S);
  }
  int rc = check_launch("batchnorm_train_fwd_f32 (stats)");
  if (rc) return rc;
  if (vec) {
    bn_normalize<true><<<grid, dim3(kThreads), 0, stream>>>(
        x, gamma, beta, running_mean, running_var, y, save_mean, save_invstd,
        ws, n, c, hw, S, momentum, eps, relu);
  } else {
    bn_normalize<false><<<grid, dim3(kThreads), 0, stream>>>(
        x, gamma, beta, running_mean, running_var, y, save_mean, save_invstd,
        ws, n, c, hw, S, momentum, eps, relu);
  }
  return check_launch("batchnorm_train_fwd_f32 (normalize)");
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the workspace is a file-scope device array.
//
// Each device the library runs on holds its own copy of `scratch`, for the
// life of the process.  On the host the array's name is only a stand-in for
// that memory: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// passed to kernels.  The first call on a device also clears the array with
// a fill kernel on the caller's stream and waits for it (that first call
// synchronises; later ones do not): the single-pass kernel's control words
// (completion count, epoch) must start at zero and its exchange slots must
// carry no tag of a future epoch.  hipo_batchnorm_noalloc_error reads (and
// clears) the array's sticky error word, the one fault signal of this path
// besides the NaN outputs.  After that, the epoch protocol keeps the array consistent from one
// call to the next, for any shape that fits; calls that overlap on one
// device (two streams) race on it.
// ---------------------------------------------------------------------------
namespace hipo {
namespace {

constexpr size_t kBnScratchBytes = size_t{4} << 20;  // 4 MiB per device
static __device__ __align__(256) unsigned char scratch[kBnScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

__global__ __launch_bounds__(256) void bn_scratch_clear(u32x4_t* __restrict__ p,
                                                       uint32_t n16) {
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n16; i += gridDim.x * 256u)
    p[i] = u32x4_t{0u, 0u, 0u, 0u};
}

// The device address of this device's scratch array, set up (and cleared on
// `stream`) by the first call on the device; nullptr after an error.
void* scratch_for_current_device(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_error("batchnorm (no-alloc): no current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] != nullptr) return g_scratch_ptr[dev];
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    set_error("batchnorm (no-alloc): the first call on a device sets up its scratch "
              "array and must not be captured; call once outside capture first");
    return nullptr;
  }
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    set_error("batchnorm (no-alloc): hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  const uint32_t n16 = static_cast<uint32_t>(kBnScratchBytes / 16);
  bn_scratch_clear<<<dim3(256), dim3(256), 0, stream>>>(static_cast<u32x4_t*>(ptr), n16);
  if (check_launch("batchnorm (no-alloc) scratch clear") != 0) return nullptr;
  // The clear completes before the address is published: a first call on
  // another stream that finds the pointer cannot start while the control
  // words are still being zeroed.
  const hipError_t se = hipStreamSynchronize(stream);
  if (se != hipSuccess) {
    (void)hipGetLastError();
    set_error("batchnorm (no-alloc): scratch clear failed: %s", hipGetErrorString(se));
    return nullptr;
  }
  g_scratch_ptr[dev] = ptr;
  return ptr;
}

}  // namespace
}  // namespace hipo

extern "C" int hipo_batchnorm_train_fwd_f32_noalloc(
    const float* x, const float* gamma, const float* beta, float* running_mean,
    float* running_var, float* y, float* save_mean, float* save_invstd,
    int64_t n, int64_t c, int64_t hw, float momentum, float eps, int relu,
    hipStream_t stream) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(n > 0 && c > 0 && hw > 0, "batchnorm: sizes must be positive");
  const size_t need = hipo_batchnorm_workspace_bytes(n, c, hw);
  HIPO_REQUIRE(need <= kBnScratchBytes,
               "batchnorm (no-alloc): this shape needs %zu bytes of workspace, more "
               "than the %zu-byte scratch array; use hipo_batchnorm_train_fwd_f32",
               need, kBnScratchBytes);
  void* ws = scratch_for_current_device(stream);
  if (ws == nullptr) return HIPO_EINVAL;
  return hipo_batchnorm_train_fwd_f32(x, gamma, beta, running_mean, running_var, y,
                                      save_mean, save_invstd, n, c, hw, momentum, eps,
                                      relu, ws, kBnScratchBytes, stream);
}

extern "C" int hipo_batchnorm_noalloc_error(int device, uint32_t* word, int clear) {
  using namespace hipo;
  clear_error();
  HIPO_REQUIRE(word != nullptr, "batchnorm_noalloc_error: null word pointer");
  *word = 0;
  HIPO_REQUIRE(device >= 0 && device < kScratchDevices,
               "batchnorm_noalloc_error: device %d out of range", device);
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[device];
  }
  if (ptr == nullptr) return 0;  // the entry point never ran on this device
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) cur = -1;
  hipError_t e = hipSetDevice(device);
  unsigned char* err = static_cast<unsigned char*>(ptr) + kBnErrorWordOffset;
  // Every kernel that may set the word has finished before it is read.
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(word, err, sizeof(uint32_t), hipMemcpyDeviceToHost);
  if (e == hipSuccess && clear && *word != 0) {
    const uint32_t zero = 0;
    e = hipMemcpy(err, &zero, sizeof(uint32_t), hipMemcpyHostToDevice);
  }
  if (cur >= 0) (void)hipSetDevice(cur);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    set_error("batchnorm_noalloc_error: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return 0;
}
