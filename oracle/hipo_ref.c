/*
 * CPU restatement of the oracle patterns -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path is libhip_oracles.so and has no CPU fallback.
 *
 * Semantics follow the eager PyTorch graphs of the build's repro modules,
 * which restate the reference's canonical repros:
 *   row mean            repros/canonical/mean_c9e1a8113328/repro.py:26
 *   bias + GELU(tanh)   repros/canonical/pointwise_2d969ac9ad59/repro.py:23-36
 *   NCHW -> NHWC        repros/canonical/pointwise_021e90d9c17d/repro.py:26-28
 *   GELU(tanh), flat    repros/canonical/pointwise_2d969ac9ad59/oracle.py:12-26
 *                       (the chain in fp32, one rounding; here in fp64)
 *   permute + clone     repros/canonical/pointwise_021e90d9c17d/repro.py:26-28
 *   ReLU + NCHW mean    repros/canonical/mean_b402ee209d0b/repro.py:24-26
 *   masked softmax      repros/canonical/amax_sum_192a3a5bd7ff/repro.py:23-44
 *   residual LayerNorm  repros/canonical/var_mean_80e7ff4dee7f/repro.py:23-39
 *   RMSNorm             repros/canonical/mean_4462ce967d63/repro.py:23-38
 *   BatchNorm train     repros/canonical/var_mean_mean_19ffdb35cc67/repro.py:23-54
 * and the corpus families the kernels generalise to:
 *   spatial mean, channels-last   repros/canonical/mean_c9e1a8113328/repro.py:26
 *   per-group bias softmax        repros/canonical/amax_sum_20ccc18dda60/repro.py:23-35
 *   T5 residual RMSNorm           repros/canonical/mean_4462ce967d63/repro.py:23-38
 *   bf16 BN + SiLU + pad (NHWC)   repros/canonical/var_mean_ceb5c315290a/repro.py:27-58
 *   bf16 BN + ReLU + mean (NCHW)  repros/canonical/var_mean_mean_19ffdb35cc67/repro.py:23-54
 *   GELU(erf) bwd + column sum    repros/canonical/sum_139a3020e8bf/repro.py:24-48
 * (paths relative to the reference tree).  Every rounding that the eager
 * graph performs on a bf16 tensor is reproduced (float arithmetic, then
 * round-to-nearest-even to bf16); reductions and transcendental functions
 * are evaluated in double, so the restatement is at least as accurate as
 * eager fp32.  Results are returned as float / bf16 bits like the kernels.
 *
 * Build: oracle/build.py (gcc -O2 -fopenmp, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* Round-to-nearest-even fp32 -> bf16; NaN stays a (quiet) NaN. */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

/* Round-to-nearest-even fp64 -> bf16 in one step (no intermediate fp32
 * rounding, which could create a false tie). */
static inline uint16_t f64_to_bf16(double d) {
  if (isnan(d)) return 0x7fc0;
  const uint16_t sign = signbit(d) ? 0x8000 : 0;
  double a = fabs(d);
  if (isinf(a)) return sign | 0x7f80;
  if (a == 0.0) return sign;
  int e;
  const double m = frexp(a, &e);               /* a = m * 2^e, m in [0.5, 1) */
  /* bf16 quantum: 2^(e-8) for normal results, 2^-133 for subnormal ones */
  int qexp = e - 8;
  if (qexp < -133) qexp = -133;
  const double scaled = ldexp(a, -qexp);       /* exact: power-of-two scaling */
  double q = floor(scaled);
  const double rem = scaled - q;               /* exact */
  if (rem > 0.5 || (rem == 0.5 && fmod(q, 2.0) == 1.0)) q += 1.0;
  (void)m;
  if (q >= 256.0) {                            /* carry into the next binade */
    q = 128.0;
    qexp += 1;
  }
  if (q >= 128.0) {
    const int field = qexp + 7 + 127;
    if (field >= 255) return sign | 0x7f80;
    return sign | (uint16_t)(field << 7) | (uint16_t)((int)q & 0x7f);
  }
  return sign | (uint16_t)q;                   /* subnormal */
}

int ref_abi_version(void) { return 1; }

int ref_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* out[r] = mean(x[r, :]) ; fp64 accumulation. */
void ref_row_mean_f32(const float* x, float* out, int64_t rows, int64_t cols,
                      int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* p = x + r * cols;
    double s = 0.0;
    for (int64_t j = 0; j < cols; ++j) s += p[j];
    out[r] = (float)(s / (double)cols);
  }
}

/* 0.5 t (1 + tanh(u)) = t / (1 + e^(-2u)), u = sqrt(2/pi) (t + 0.044715 t^3):
 * the second form does not cancel in the negative tail, where 1 + tanh(u)
 * would lose every digit in double below t ~ -5.  Specials: gelu(+inf) =
 * +inf, gelu(-inf) = NaN (as eager's -inf * 0), NaN -> NaN. */
static inline double gelu_tanh(double t) {
  const double k = 0.7978845608028654; /* sqrt(2/pi) */
  const double u = k * (t + 0.044715 * t * t * t);
  return t / (1.0 + exp(-2.0 * u));
}

/*
 * out (NHWC, bf16 bits) = bf16(gelu_tanh(t)), t = x[n,c,hw] + bias[c].
 * round_t != 0 rounds t to bf16 first (what eager's bf16 add stores).
 */
void ref_bias_gelu_nchw_to_nhwc_bf16(const uint16_t* x, const uint16_t* bias,
                                     uint16_t* out, int64_t n, int64_t c,
                                     int64_t hw, int round_t, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static) collapse(2)
  for (int64_t i = 0; i < n; ++i) {
    for (int64_t p = 0; p < hw; ++p) {
      uint16_t* o = out + (i * hw + p) * c;
      for (int64_t ch = 0; ch < c; ++ch) {
        float t = bf16_to_f32(x[(i * c + ch) * hw + p]) + bf16_to_f32(bias[ch]);
        if (round_t) t = round_bf16(t);
        o[ch] = f64_to_bf16(gelu_tanh((double)t));
      }
    }
  }
}

/*
 * s = x * scale + bias[b / heads, q, :] (exact in fp64: no rounding of the
 * scores, as the reference's Triton oracle forms them in fp32 --
 * amax_sum_20ccc18dda60/oracle.py:44-46; eager's bf16 roundings of x * scale
 * and of the sum are exact for the causal softmax's power-of-two scale and
 * 0 / -inf mask); out = bf16(softmax(s)) with the max, exp and sum in fp64.
 * x/out [batch, q, k]; the bias row of
 * (b, q) starts at (b / heads) * bias_batch_stride + q * bias_row_stride
 * elements.  The masked softmax is the case batch_stride = 0, heads = 1.
 */
void ref_scaled_bias_softmax_bf16(const uint16_t* x, const uint16_t* mask,
                                  uint16_t* out, int64_t batch, int64_t q,
                                  int64_t k, int64_t mask_stride,
                                  int64_t mask_batch_stride, int64_t heads,
                                  float scale, int threads) {
  const int64_t rows = batch * q;
  if (k <= 0) return;
#pragma omp parallel num_threads(threads)
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)k); /* per thread */
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const uint16_t* xr = x + r * k;
      const uint16_t* mr =
          mask + ((r / q) / heads) * mask_batch_stride + (r % q) * mask_stride;
      double m = -INFINITY;
      for (int64_t j = 0; j < k; ++j) {
        const double v = (double)bf16_to_f32(xr[j]) * (double)scale + bf16_to_f32(mr[j]);
        s[j] = v;
        if (isnan(v) || isnan(m)) {
          m = NAN; /* amax propagates NaN */
        } else if (v > m) {
          m = v;
        }
      }
      double sum = 0.0;
      for (int64_t j = 0; j < k; ++j) {
        s[j] = exp(s[j] - m);
        sum += s[j];
      }
      uint16_t* o = out + r * k;
      for (int64_t j = 0; j < k; ++j) o[j] = f64_to_bf16(s[j] / sum);
    }
    free(s);
  }
}

void ref_scaled_masked_softmax_bf16(const uint16_t* x, const uint16_t* mask,
                                    uint16_t* out, int64_t batch, int64_t q,
                                    int64_t k, int64_t mask_stride, float scale,
                                    int threads) {
  ref_scaled_bias_softmax_bf16(x, mask, out, batch, q, k, mask_stride, 0, 1, scale,
                               threads);
}

/*
 * h = bf16(x + residual); mean, var (population) of h in fp64;
 * rstd = 1/sqrt(var + eps); y = bf16((h - mean) * rstd * gamma + beta).
 */
void ref_residual_layernorm_bf16(const uint16_t* x, const uint16_t* res,
                                 const uint16_t* gamma, const uint16_t* beta,
                                 uint16_t* h, uint16_t* y, float* mean_out,
                                 float* rstd_out, int64_t rows, int64_t cols,
                                 float eps, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t base = r * cols;
    double s = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      const uint16_t hb = f32_to_bf16(bf16_to_f32(x[base + j]) + bf16_to_f32(res[base + j]));
      h[base + j] = hb;
      s += bf16_to_f32(hb);
    }
    const double mean = s / (double)cols;
    double q = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      const double d = bf16_to_f32(h[base + j]) - mean;
      q += d * d;
    }
    const double rstd = 1.0 / sqrt(q / (double)cols + (double)eps);
    for (int64_t j = 0; j < cols; ++j) {
      const double v = (bf16_to_f32(h[base + j]) - mean) * rstd *
                           bf16_to_f32(gamma[j]) + bf16_to_f32(beta[j]);
      y[base + j] = f64_to_bf16(v);
    }
    mean_out[r] = (float)mean;
    rstd_out[r] = (float)rstd;
  }
}

/* rstd = 1/sqrt(mean(x^2) + eps); y = bf16(x * rstd * gamma). */
void ref_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma, uint16_t* y,
                      float* rstd_out, int64_t rows, int64_t cols, float eps,
                      int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t base = r * cols;
    double q = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      const double v = bf16_to_f32(x[base + j]);
      q += v * v;
    }
    const double rstd = 1.0 / sqrt(q / (double)cols + (double)eps);
    for (int64_t j = 0; j < cols; ++j) {
      const double v = bf16_to_f32(x[base + j]) * rstd * bf16_to_f32(gamma[j]);
      y[base + j] = f64_to_bf16(v);
    }
    rstd_out[r] = (float)rstd;
  }
}

/*
 * BatchNorm training forward over (N, H, W) of NCHW fp32, fp64 statistics:
 *   save_mean = mean; save_invstd = 1/sqrt(var + eps)   (var: correction 0)
 *   y = relu?((x - mean) * invstd * gamma + beta)
 *   running_mean = (1 - m) running_mean + m mean
 *   running_var  = (1 - m) running_var  + m var * cnt / (cnt - 1)
 */
void ref_batchnorm_train_f32(const float* x, const float* gamma,
                             const float* beta, float* running_mean,
                             float* running_var, float* y, float* save_mean,
                             float* save_invstd, int64_t n, int64_t c,
                             int64_t hw, float momentum, float eps, int relu,
                             int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t ch = 0; ch < c; ++ch) {
    const double cnt = (double)n * (double)hw;
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const float* p = x + (i * c + ch) * hw;
      for (int64_t j = 0; j < hw; ++j) s += p[j];
    }
    const double mean = s / cnt;
    double q = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const float* p = x + (i * c + ch) * hw;
      for (int64_t j = 0; j < hw; ++j) {
        const double d = p[j] - mean;
        q += d * d;
      }
    }
    const double var = q / cnt;
    const double invstd = 1.0 / sqrt(var + (double)eps);
    const double g = gamma[ch], b = beta[ch];
    for (int64_t i = 0; i < n; ++i) {
      const float* p = x + (i * c + ch) * hw;
      float* o = y + (i * c + ch) * hw;
      for (int64_t j = 0; j < hw; ++j) {
        double v = (p[j] - mean) * invstd * g + b;
        if (relu && !(v > 0.0)) v = isnan(v) ? v : 0.0;
        o[j] = (float)v;
      }
    }
    save_mean[ch] = (float)mean;
    save_invstd[ch] = (float)invstd;
    const double mom = momentum;
    const double unbiased = cnt > 1.0 ? q / (cnt - 1.0) : NAN;
    running_mean[ch] = (float)(mom * mean + (1.0 - mom) * running_mean[ch]);
    running_var[ch] = (float)(mom * unbiased + (1.0 - mom) * running_var[ch]);
  }
}

/*
 * Spatial mean of a channels-last bf16 tensor, physical [n, p, c]:
 * out[n, c] = bf16(sum_p x / p), the sum in fp64.
 */
void ref_spatial_mean_nhwc_bf16(const uint16_t* x, uint16_t* out, int64_t n,
                                int64_t p, int64_t c, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < n * c; ++i) {
    const int64_t img = i / c, ch = i % c;
    const uint16_t* src = x + img * p * c + ch;
    double s = 0.0;
    for (int64_t j = 0; j < p; ++j) s += bf16_to_f32(src[j * c]);
    out[i] = f64_to_bf16(s / (double)p);
  }
}

/*
 * RMSNorm with an optional residual and output scale, in the two eager op
 * orders:  h = residual ? bf16(x + residual) : x;  rstd = 1/sqrt(mean(h^2)
 * + eps) (fp64);  mode 0: y = bf16(h * rstd * gamma * scale) (one rounding,
 * torch rms_norm);  mode 1 (HF T5): t = bf16(h * rstd); u = bf16(gamma * t);
 * y = scale == 1 ? u : bf16(u * scale).  residual may be NULL.
 */
void ref_rmsnorm_ex_bf16(const uint16_t* x, const uint16_t* res, const uint16_t* gamma,
                         uint16_t* y, float* rstd_out, int64_t rows, int64_t cols,
                         float eps, float scale, int mode, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t base = r * cols;
    double q = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      const float a = bf16_to_f32(x[base + j]);
      const double h = res ? round_bf16(a + bf16_to_f32(res[base + j])) : a;
      q += h * h;
    }
    const double rstd = 1.0 / sqrt(q / (double)cols + (double)eps);
    for (int64_t j = 0; j < cols; ++j) {
      const float a = bf16_to_f32(x[base + j]);
      const double h = res ? round_bf16(a + bf16_to_f32(res[base + j])) : a;
      const double g = bf16_to_f32(gamma[j]);
      if (mode == 0) {
        y[base + j] = f64_to_bf16(h * rstd * g * (double)scale);
      } else {
        const double t = bf16_to_f32(f64_to_bf16(h * rstd));
        const double u = bf16_to_f32(f64_to_bf16(g * t));
        y[base + j] = scale == 1.0f ? f64_to_bf16(u) : f64_to_bf16(u * (double)scale);
      }
    }
    if (rstd_out) rstd_out[r] = (float)rstd;
  }
}

/* act(bf16(((x - mean) * rstd) * gamma + beta)) of the bf16 BN graphs, in
 * fp64 with the graph's bf16 rounding; act 0 none, 1 ReLU, 2 SiLU (rounded
 * to bf16 again). */
static inline double bn_bf16_act(double xv, double mean, double rstd, double g, double b,
                                 int act) {
  double t = bf16_to_f32(f64_to_bf16((xv - mean) * rstd * g + b));
  if (act == 1) {
    t = t < 0.0 ? 0.0 : t;
  } else if (act == 2) {
    t = bf16_to_f32(f64_to_bf16(t / (1.0 + exp(-t))));
  }
  return t;
}

/* Per-channel statistics, save_* and running statistics of the bf16 BN
 * graphs: var with correction 0 in fp64; save_rstd = 1/sqrt(float(var) +
 * eps); running_mean = mean*m + rm*(1-m); running_var = var*var_scale*m +
 * rv*(1-m).  at(i, j) addresses channel element j of channel i's `cnt`. */
static void bn_bf16_stats(const uint16_t* x, int64_t cnt, int64_t c, int nhwc, int64_t n,
                          int64_t hw, float momentum, float eps, float var_scale,
                          float* running_mean, float* running_var, float* save_mean,
                          float* save_rstd, double* mean_out, double* rstd_out, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t ch = 0; ch < c; ++ch) {
    double s = 0.0;
    for (int64_t i = 0; i < cnt; ++i) {
      const int64_t idx = nhwc ? i * c + ch : ((i / hw) * c + ch) * hw + i % hw;
      s += bf16_to_f32(x[idx]);
    }
    const double mean = s / (double)cnt;
    double q = 0.0;
    for (int64_t i = 0; i < cnt; ++i) {
      const int64_t idx = nhwc ? i * c + ch : ((i / hw) * c + ch) * hw + i % hw;
      const double d = bf16_to_f32(x[idx]) - mean;
      q += d * d;
    }
    const double var = q / (double)cnt;
    const double rstd = 1.0 / sqrt((double)(float)var + (double)eps);
    save_mean[ch] = (float)mean;
    save_rstd[ch] = (float)rstd;
    mean_out[ch] = (float)mean;
    rstd_out[ch] = (float)rstd;
    const double m = momentum;
    running_mean[ch] = (float)(mean * m + running_mean[ch] * (1.0 - m));
    running_var[ch] = (float)(var * var_scale * m + running_var[ch] * (1.0 - m));
  }
  (void)n;
}

/*
 * Channels-last bf16 BatchNorm training forward + activation + zero pad of
 * the bottom / right border: x physical [n, h, w, c]; out physical
 * [n, h + pad_bottom, w + pad_right, c].
 */
void ref_batchnorm_nhwc_act_pad_bf16(const uint16_t* x, const float* gamma,
                                     const float* beta, float* running_mean,
                                     float* running_var, float* save_mean,
                                     float* save_rstd, uint16_t* out, int64_t n,
                                     int64_t h, int64_t w, int64_t c, int64_t pad_bottom,
                                     int64_t pad_right, float momentum, float eps,
                                     float var_scale, int act, int threads) {
  double* mean = (double*)malloc(sizeof(double) * (size_t)c);
  double* rstd = (double*)malloc(sizeof(double) * (size_t)c);
  bn_bf16_stats(x, n * h * w, c, 1, n, h * w, momentum, eps, var_scale, running_mean,
                running_var, save_mean, save_rstd, mean, rstd, threads);
  const int64_t ho = h + pad_bottom, wo = w + pad_right;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t o = 0; o < n * ho * wo; ++o) {
    const int64_t img = o / (ho * wo), rem = o % (ho * wo), y = rem / wo, xw = rem % wo;
    for (int64_t ch = 0; ch < c; ++ch) {
      double v = 0.0;
      if (y < h && xw < w) {
        const double xv = bf16_to_f32(x[((img * h + y) * w + xw) * c + ch]);
        v = bn_bf16_act(xv, mean[ch], rstd[ch], gamma[ch], beta[ch], act);
      }
      out[o * c + ch] = f64_to_bf16(v);
    }
  }
  free(mean);
  free(rstd);
}

/*
 * NCHW bf16 BatchNorm training forward + activation + mean over H, W:
 * out[n, c] = bf16(mean_hw act(...)) (fp64 sum).
 */
void ref_batchnorm_nchw_act_mean_bf16(const uint16_t* x, const float* gamma,
                                      const float* beta, float* running_mean,
                                      float* running_var, float* save_mean,
                                      float* save_rstd, uint16_t* out, int64_t n,
                                      int64_t c, int64_t hw, float momentum, float eps,
                                      float var_scale, int act, int threads) {
  double* mean = (double*)malloc(sizeof(double) * (size_t)c);
  double* rstd = (double*)malloc(sizeof(double) * (size_t)c);
  bn_bf16_stats(x, n * hw, c, 0, n, hw, momentum, eps, var_scale, running_mean,
                running_var, save_mean, save_rstd, mean, rstd, threads);
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < n * c; ++i) {
    const int64_t ch = i % c;
    const uint16_t* seg = x + i * hw;
    double s = 0.0;
    for (int64_t j = 0; j < hw; ++j)
      s += bn_bf16_act(bf16_to_f32(seg[j]), mean[ch], rstd[ch], gamma[ch], beta[ch], act);
    out[i] = f64_to_bf16(s / (double)hw);
  }
  free(mean);
  free(rstd);
}

/* y = bf16(gelu_tanh(x)) of n bf16 values: fp64, one rounding. */
void ref_gelu_tanh_bf16(const uint16_t* x, uint16_t* y, int64_t n, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = f64_to_bf16(gelu_tanh((double)bf16_to_f32(x[i])));
}

/* y = (float)gelu_tanh(x) of n fp32 values: fp64, one rounding. */
void ref_gelu_tanh_f32(const float* x, float* y, int64_t n, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < n; ++i) y[i] = (float)gelu_tanh((double)x[i]);
}

/* y[b, c, r] = x[b, r, c] for elements of es bytes (any es). */
void ref_transpose_last2(const void* x, void* y, int64_t batch, int64_t rows, int64_t cols,
                         int es, int threads) {
  const unsigned char* xs = (const unsigned char*)x;
  unsigned char* ys = (unsigned char*)y;
#pragma omp parallel for num_threads(threads) schedule(static) collapse(2)
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t r = 0; r < rows; ++r) {
      for (int64_t c = 0; c < cols; ++c) {
        memcpy(ys + ((b * cols + c) * rows + r) * es, xs + ((b * rows + r) * cols + c) * es,
               (size_t)es);
      }
    }
  }
}

/* out[r] = bf16(sum_j act(x[r, j]) / cols), fp64 sum; act = ReLU (NaN kept)
 * when relu != 0. */
void ref_row_mean_bf16(const uint16_t* x, uint16_t* out, int64_t rows, int64_t cols,
                       int relu, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* p = x + r * cols;
    double s = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
      double v = bf16_to_f32(p[j]);
      if (relu && v < 0.0) v = 0.0;
      s += v;
    }
    out[r] = f64_to_bf16(s / (double)cols);
  }
}

/* d(t) = Phi(t) + t phi(t), the derivative of GELU(erf) t Phi(t), in fp64
 * (Phi through erfc, so the negative tail does not cancel) and rounded once
 * to fp32; inf and NaN give NaN (as eager's t * exp(-t^2 / 2) = inf * 0). */
static inline float gelu_erf_grad_f32(float t) {
  const double td = (double)t;
  const double cdf = 0.5 * erfc(-td * 0.70710678118654752440);
  const double pdf = exp(-0.5 * td * td) * 0.39894228040143267794; /* 1 / sqrt(2 pi) */
  return (float)(cdf + td * pdf);
}

/* d[i] = the fp32 d(t) above for n bf16 inputs t. */
void ref_gelu_erf_grad_f32(const uint16_t* x, float* d, int64_t n, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < n; ++i) d[i] = gelu_erf_grad_f32(bf16_to_f32(x[i]));
}

/* GELU(erf) backward and the column sum of its output (the graph of
 * repros/canonical/sum_139a3020e8bf/repro.py:24-48):
 *   y[r, c]   = bf16(g[r, c] * d(x[r, c]))   (one fp32 product)
 *   colsum[c] = bf16(sum_r y[r, c]), fp64 sum, one rounding, stored as fp32.
 * The fp64 sums run over fixed blocks of 1024 rows (in parallel) and then
 * over the blocks in order: the result does not depend on the thread count. */
void ref_gelu_erf_bwd_colsum_bf16(const uint16_t* g, const uint16_t* x, uint16_t* y,
                                  float* colsum, int64_t rows, int64_t cols, int threads) {
  const int64_t kBlock = 1024;
  const int64_t nblk = (rows + kBlock - 1) / kBlock;
  double* part = (double*)calloc((size_t)(nblk > 0 ? nblk : 1) * (size_t)(cols > 0 ? cols : 1),
                                 sizeof(double));
  if (part == NULL) abort();
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (int64_t b = 0; b < nblk; ++b) {
    double* acc = part + b * cols;
    const int64_t r1 = (b + 1) * kBlock < rows ? (b + 1) * kBlock : rows;
    for (int64_t r = b * kBlock; r < r1; ++r) {
      for (int64_t c = 0; c < cols; ++c) {
        const int64_t i = r * cols + c;
        y[i] = f32_to_bf16(bf16_to_f32(g[i]) * gelu_erf_grad_f32(bf16_to_f32(x[i])));
        acc[c] += bf16_to_f32(y[i]);
      }
    }
  }
  for (int64_t c = 0; c < cols; ++c) {
    double s = 0.0;
    for (int64_t b = 0; b < nblk; ++b) s += part[b * cols + c];
    colsum[c] = bf16_to_f32(f64_to_bf16(s));
  }
  free(part);
}
