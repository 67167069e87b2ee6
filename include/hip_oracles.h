/*
 * hip_oracles.h -- C ABI of libhip_oracles.so, the MI355X (gfx950) kernel
 * library behind the gfx950 oracle registrations.
 *
 * In better-benchmark an oracle is `oracle_forward(inputs, **cfg)` in a
 * canonical repro's oracle.py, registered with `@oracle_impl(...)`
 * (reference: oracle_harness.py:468-549); its body launches Triton kernels.
 * Each entry point below replaces one such body: the Python oracle
 * allocates the outputs with torch, then calls here with raw device pointers,
 * sizes and the caller's HIP stream.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers.  bf16 tensors are passed as uint16_t*
 *     (raw bfloat16 bit patterns).  Tensors are dense and row-major
 *     (contiguous) unless a stride argument says otherwise.
 *   - `stream` is the caller's stream (torch.cuda.current_stream()); every
 *     launch goes on it.  Calls only enqueue work: no allocation, no
 *     synchronisation, no host<->device copies, so they are safe under
 *     hipStreamBeginCapture / torch.cuda.graph.
 *   - Return 0 on success.  Non-zero is a hipError_t from the launch, or
 *     HIPO_EINVAL (argument check failed before anything was launched).
 *     hipo_last_error() then holds a message (per calling thread).
 *   - Re-entrant.  The only global state is a per-device cache of device
 *     properties, filled on first use.
 */
#ifndef HIP_ORACLES_H_
#define HIP_ORACLES_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HIPO_ABI_VERSION 4
#define HIPO_EINVAL 1000

/* ABI version of the loaded library (HIPO_ABI_VERSION at build time). */
int hipo_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char* hipo_last_error(void);

/*
 * Row mean: out[r] = mean(x[r, 0:cols]) in fp32.
 * x is [rows, cols] with row stride `row_stride` elements (>= cols).
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/mean_c9e1a8113328/oracle.py:95 (_spatial_mean_row_kernel,
 * same file :45) for the row-reduction form `x.mean(dim=-1)`.
 */
int hipo_row_mean_f32(const float* x, float* out, int64_t rows, int64_t cols,
                      int64_t row_stride, hipStream_t stream);

/*
 * Channel bias + GELU(tanh) + NCHW -> NHWC:
 *   t = bf16(x[n,c,hw] + bias[c])       (eager order: the add rounds to bf16)
 *   y = 0.5 t (1 + tanh(sqrt(2/pi) (t + 0.044715 t^3)))
 *   out[n,hw,c] = bf16(y), correctly rounded (t is bf16: a table of the
 *                 exactly rounded results by bit pattern)
 * x is contiguous NCHW [n, c, hw]; out is the same logical tensor stored
 * channels-last (physical [n, hw, c]).
 * Replaces the Triton bodies of oracle_forward in
 * repros/canonical/pointwise_2d969ac9ad59/oracle.py:47 (tanh GELU) and
 * repros/canonical/pointwise_021e90d9c17d/oracle.py:58 (permute + clone),
 * fused into one pass.
 */
int hipo_bias_gelu_nchw_to_nhwc_bf16(const uint16_t* x, const uint16_t* bias,
                                     uint16_t* out, int64_t n, int64_t c,
                                     int64_t hw, hipStream_t stream);

/*
 * Scaled, additively masked softmax over the last dim (bf16 in/out):
 *   s[b,q,k] = fma(x[b,q,k], scale, mask[q,k])     (fp32 scores)
 *   out[b,q,:] = bf16(softmax_fp32(s[b,q,:]))
 * (eager's bf16 roundings of x * scale and of the sum are exact for a
 * power-of-two scale and a 0 / -inf mask, the causal softmax.)
 * x/out are [batch, q, k] contiguous; mask is [q, k] with row stride
 * `mask_row_stride` elements, broadcast over batch.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/amax_sum_20ccc18dda60/oracle.py:63
 * (_broadcast_add_softmax_kernel, same file :12), and -- with q = 1, one
 * zero mask row and scale 1 -- the plain softmax of
 * repros/canonical/amax_sum_fa4cc85fe5ad/oracle.py:68 (_bf16_softmax_kernel,
 * same file :12).
 */
int hipo_scaled_masked_softmax_bf16(const uint16_t* x, const uint16_t* mask,
                                    uint16_t* out, int64_t batch, int64_t q,
                                    int64_t k, int64_t mask_row_stride,
                                    float scale, hipStream_t stream);

/*
 * Residual add + LayerNorm forward over the last dim (bf16 in/out):
 *   h = bf16(x + residual);  mean, var = fp32 stats of h (population var)
 *   rstd = 1/sqrt(var + eps);  y = bf16((h - mean) * rstd * gamma + beta)
 * x, residual, h, y are [rows, cols] contiguous; gamma, beta are [cols];
 * mean, rstd are fp32 [rows].  h, mean and rstd may be NULL: that output is
 * not written (the reference's var_mean_80e7ff4dee7f returns y only).
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/var_mean_80e7ff4dee7f/oracle.py:122
 * (_residual_layernorm_kernel, same file :51), and of the residual-LayerNorm
 * families var_mean_0ada225c0a04, var_mean_96edf0542ecd,
 * var_mean_f4578c128d74, var_mean_b19e82f2a47b, var_mean_393456b916a6 and
 * var_mean_45f7dfd4a983 (oracle.py, oracle_forward).
 */
int hipo_residual_layernorm_bf16(const uint16_t* x, const uint16_t* residual,
                                 const uint16_t* gamma, const uint16_t* beta,
                                 uint16_t* h, uint16_t* y, float* mean,
                                 float* rstd, int64_t rows, int64_t cols,
                                 float eps, hipStream_t stream);

/*
 * RMSNorm forward over the last dim (bf16 in/out):
 *   rstd = 1/sqrt(mean(x^2) + eps)   (fp32)
 *   y = bf16(x * rstd * gamma)       (fp32 arithmetic, one rounding)
 * x, y are [rows, cols] contiguous; gamma is [cols]; rstd is fp32 [rows].
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/mean_4462ce967d63/oracle.py:65.
 */
int hipo_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma, uint16_t* y,
                      float* rstd, int64_t rows, int64_t cols, float eps,
                      hipStream_t stream);

/*
 * RMSNorm with the options the corpus variants use:
 *   h = residual ? bf16(x + residual) : x       (the eager bf16 add)
 *   rstd = 1/sqrt(mean(h^2) + eps)             (fp32)
 *   mode 0: y = bf16(h * rstd * gamma * scale)  (torch rms_norm, one rounding)
 *   mode 1: t = bf16(h * rstd); u = bf16(gamma * t);
 *           y = scale == 1 ? u : bf16(u * scale)   (HF T5 LayerNorm op order)
 * residual, h and rstd may be NULL (h, the bf16 sum, only with a
 * residual).  Shapes as hipo_rmsnorm_bf16.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/mean_4462ce967d63/oracle.py:65 (T5: residual, eps 1e-6,
 * mode 1, scale 0.04419417382415922) and of the residual-RMSNorm families
 * mean_f08c75b5f21f, mean_db9733790220, mean_8818e35b12aa,
 * mean_c033ad4c69ca, mean_f21cc667fe83 (mode 0), mean_426e2409482e,
 * mean_4dace6865eee, mean_bf2ed36e56df, mean_d28c6a07654f and
 * mean_41e8bba10b8b (oracle.py, oracle_forward).
 */
int hipo_rmsnorm_ex_bf16(const uint16_t* x, const uint16_t* residual,
                         const uint16_t* gamma, uint16_t* h, uint16_t* y, float* rstd,
                         int64_t rows, int64_t cols, float eps, float scale,
                         int mode, hipStream_t stream);

/*
 * Softmax over the last dim with an additive bias shared by groups of
 * `heads` consecutive batch entries:
 *   s[b,q,k] = fma(x[b,q,k], scale, bias[b / heads][q, k])   (fp32 scores,
 *              as the reference's Triton oracle builds them)
 *   out[b,q,:] = bf16(softmax_fp32(s[b,q,:]))
 * bias row of (b, q): bias + (b / heads) * bias_batch_stride
 *                          + q * bias_row_stride   (elements).
 * hipo_scaled_masked_softmax_bf16 is the case bias_batch_stride = 0.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/amax_sum_20ccc18dda60/oracle.py:63 (x viewed
 * [64, 16, 256, 256] + bias [64, 1, 256, 256]: heads = 16, scale = 1).
 */
int hipo_scaled_bias_softmax_bf16(const uint16_t* x, const uint16_t* bias,
                                  uint16_t* out, int64_t batch, int64_t q,
                                  int64_t k, int64_t bias_row_stride,
                                  int64_t bias_batch_stride, int64_t heads,
                                  float scale, hipStream_t stream);

/*
 * Bytes of fp32 workspace hipo_spatial_mean_nhwc_bf16 needs (0: none).
 */
size_t hipo_spatial_mean_workspace_bytes(int64_t n, int64_t hw, int64_t c);

/*
 * Spatial mean of a channels-last bf16 tensor (a reduction over a
 * non-innermost axis):
 *   out[n, c] = bf16(sum_p x[n, p, c] / hw)     (fp32 accumulation)
 * x is [n, c, h, w] stored channels-last, i.e. physical [n, hw, c] with c
 * contiguous; out is [n, c] contiguous ([n, c, 1, 1] keepdim).  `workspace`
 * holds fp32 partial sums when the kernel splits positions; size from
 * hipo_spatial_mean_workspace_bytes (may be NULL when that is 0).
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/mean_c9e1a8113328/oracle.py:95
 * (_spatial_mean_cl_kernel, same file :11).
 */
int hipo_spatial_mean_nhwc_bf16(const uint16_t* x, uint16_t* out, int64_t n,
                                int64_t hw, int64_t c, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);

/*
 * BatchNorm training forward on bf16 activations, fp32 statistics, in the
 * op order of the reference's bf16 BN graphs:
 *   mean[c], var[c] = var_mean(fp32(x), dims (0, 2, 3), correction 0)
 *   save_mean = mean;  save_rstd = 1 / sqrt(var + eps)
 *   y = act(bf16(((x - mean) * save_rstd) * gamma + beta))     (fp32 ops)
 *       act: 0 none, 1 ReLU, 2 SiLU (t / (1 + e^-t), rounded to bf16)
 *   running_mean = mean * momentum + running_mean * (1 - momentum)
 *   running_var  = (var * var_scale) * momentum
 *                  + running_var * (1 - momentum)             (in place)
 * var_scale is the graph's Bessel constant (N/(N-1) at the shape the graph
 * was captured at); it is applied as given.  gamma, beta, running_*,
 * save_* are fp32 [c].  The statistics pass writes (mean, M2) per slice and
 * channel into `workspace` (16-byte aligned, at least the size the matching
 * *_workspace_bytes call returns; no initialisation needed); calls that
 * share a workspace must be ordered.  Deterministic (fixed merge order).
 */

/* Workspace bytes of hipo_batchnorm_nhwc_act_pad_bf16 (0: empty shape). */
size_t hipo_batchnorm_nhwc_workspace_bytes(int64_t n, int64_t h, int64_t w, int64_t c);

/*
 * x is [n, c, h, w] stored channels-last (physical [n, h, w, c]); out is
 * [n, c, h + pad_bottom, w + pad_right] stored channels-last, y in the
 * top-left h x w window and zeros in the padding.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/var_mean_ceb5c315290a/oracle.py:238 (split-K statistics,
 * then the normalise + SiLU + pad epilogue; eps 1e-3, SiLU, pad 1).
 */
int hipo_batchnorm_nhwc_act_pad_bf16(const uint16_t* x, const float* gamma,
                                     const float* beta, float* running_mean,
                                     float* running_var, float* save_mean,
                                     float* save_rstd, uint16_t* out, int64_t n,
                                     int64_t h, int64_t w, int64_t c,
                                     int64_t pad_bottom, int64_t pad_right,
                                     float momentum, float eps, float var_scale,
                                     int act, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes of hipo_batchnorm_nchw_act_mean_bf16 (0: empty shape). */
size_t hipo_batchnorm_nchw_mean_workspace_bytes(int64_t n, int64_t c, int64_t hw);

/*
 * x is contiguous NCHW [n, c, hw]; out[n, c] = bf16(mean over hw of y)
 * (fp32 sum), a contiguous [n, c] bf16 tensor.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/var_mean_mean_19ffdb35cc67/oracle.py:167 (one CTA per
 * channel, then the normalise + ReLU + spatial-mean epilogue; eps 1e-5).
 */
int hipo_batchnorm_nchw_act_mean_bf16(const uint16_t* x, const float* gamma,
                                      const float* beta, float* running_mean,
                                      float* running_var, float* save_mean,
                                      float* save_rstd, uint16_t* out, int64_t n,
                                      int64_t c, int64_t hw, float momentum,
                                      float eps, float var_scale, int act,
                                      void* workspace, size_t workspace_bytes,
                                      hipStream_t stream);

/*
 * Bytes of device workspace hipo_batchnorm_train_fwd_f32 needs for this
 * shape (0 if a size is not positive).
 */
size_t hipo_batchnorm_workspace_bytes(int64_t n, int64_t c, int64_t hw);

/*
 * BatchNorm training forward over dims (0, 2, 3) of NCHW fp32, fused with
 * the affine transform, an optional ReLU and the running-stat update:
 *   mean[c], var[c] = population stats of x[:, c, :]   (correction 0)
 *   save_mean = mean;  save_invstd = 1/sqrt(var + eps)
 *   y = relu?((x - mean) * save_invstd * gamma + beta)
 *   running_mean = (1 - momentum) running_mean + momentum mean
 *   running_var  = (1 - momentum) running_var
 *                  + momentum var * count / (count - 1)     (in place)
 * x, y are contiguous [n, c, hw]; gamma, beta, running_*, save_* are [c].
 * Channels of at most 16384 values (n * hw) run as one launch with a
 * workgroup per channel that holds it in registers (reads x once, uses no
 * workspace); larger ones as one persistent kernel that reads x once (HW a
 * multiple of 4, 16-byte aligned x / y, x under 4 GiB), others as two
 * split-K launches that read x twice.
 * `workspace` is caller-allocated device memory, 8-byte aligned, of at
 * least hipo_batchnorm_workspace_bytes(n, c, hw) bytes.  It must be
 * zero-filled before its first use and then passed unmodified to later
 * calls: the single-pass kernel keeps its cross-workgroup exchange state
 * there (a completion count, a launch epoch, tagged partial statistics).
 * Calls that share a workspace must be ordered (one stream); bytes 8..11
 * hold a sticky error word, nonzero after an exchange wait timed out (the
 * affected channels' outputs are then NaN).
 * Replaces the Triton bodies of oracle_forward in
 * repros/canonical/var_mean_mean_19ffdb35cc67/oracle.py:167 (one CTA per
 * channel) and repros/canonical/var_mean_ceb5c315290a/oracle.py:238
 * (split-K sum/sum-of-squares, then an epilogue that re-reads x).
 */
int hipo_batchnorm_train_fwd_f32(const float* x, const float* gamma,
                                 const float* beta, float* running_mean,
                                 float* running_var, float* y,
                                 float* save_mean, float* save_invstd,
                                 int64_t n, int64_t c, int64_t hw,
                                 float momentum, float eps, int relu,
                                 void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/*
 * hipo_batchnorm_train_fwd_f32 without a caller workspace and without any
 * allocation: no counterpart in the reference.  For callers that cannot
 * allocate device memory or pass a workspace (code under hipGraph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * semantics, kernels and results as hipo_batchnorm_train_fwd_f32, minus the
 * workspace: it uses a 4 MiB file-scope device array per device instead,
 * held until the process ends.  Shapes whose
 * hipo_batchnorm_workspace_bytes(n, c, hw) exceeds 4 MiB are rejected with
 * HIPO_EINVAL (config [128, 256, 56, 56] needs about 96 KiB).  The first
 * call on a device looks up the array's address and clears it with a fill
 * kernel on `stream`; that first call must not be under stream capture
 * (HIPO_EINVAL), later ones may be.  Every call on a device shares that
 * device's array: calls that overlap on one device (several streams) race
 * and must not be issued.
 */
int hipo_batchnorm_train_fwd_f32_noalloc(const float* x, const float* gamma,
                                         const float* beta, float* running_mean,
                                         float* running_var, float* y,
                                         float* save_mean, float* save_invstd,
                                         int64_t n, int64_t c, int64_t hw,
                                         float momentum, float eps, int relu,
                                         hipStream_t stream);

/*
 * The sticky error word of the allocation-free path's static scratch array
 * on `device`: nonzero once an exchange wait of the single-pass kernel
 * timed out there (that call's outputs and running statistics are then
 * NaN).  *word = 0 if hipo_batchnorm_train_fwd_f32_noalloc never ran on the
 * device.  Waits for the device's work to finish (a host query, not a launch:
 * never call it under stream capture); with `clear`, a nonzero word is reset
 * to zero.  No counterpart in the reference: the fault channel of the
 * allocation-free entry point, whose workspace the caller cannot inspect.
 */
int hipo_batchnorm_noalloc_error(int device, uint32_t* word, int clear);

/*
 * Flat stream copy (a measurement yardstick, not an oracle): reads
 * read_bytes from src and writes write_bytes to dst in one launch with the
 * oracle kernels' access style (16-byte non-temporal accesses, 1 KiB per
 * wave, one-shot grid in memory order); chunk i of dst receives chunk i of
 * src where both exist.  Sizes are multiples of 1024 (write_bytes >= 1024),
 * pointers 16-byte aligned.  The time of this copy at a config's read and
 * write bytes is the ceiling the config's kernel is compared with.
 * Counterpart of the reference's memcopy speed-of-light construction
 * (repro_harness.py:952-958, an fp32 add(src, 1, out=dst) over the same
 * bytes), written for MI355X with the stores that kernel lacks.
 */
int hipo_flat_copy(const void* src, int64_t read_bytes, void* dst,
                   int64_t write_bytes, hipStream_t stream);

/*
 * Yardstick for two-input, two-output streaming kernels (the residual
 * LayerNorm: x, residual -> h, y): copies bytes of src0 to dst0 and of src1
 * to dst1 in one launch, each wave moving one 1 KiB chunk of all four
 * buffers with 16-byte non-temporal accesses.  bytes: a positive multiple
 * of 1024; pointers 16-byte aligned.  No counterpart in the reference (its
 * memcopy SOL is one stream each way, repro_harness.py:952-958); used only
 * to price a kernel's access pattern.
 */
int hipo_flat_copy2(const void* src0, const void* src1, void* dst0, void* dst1,
                    int64_t bytes, hipStream_t stream);

/*
 * Yardstick for the single-pass BatchNorm (hipo_batchnorm_train_fwd_f32's
 * fused kernel): y = x for fp32 [n, c, hw] NCHW, with that kernel's exact
 * access pattern -- the same slabs and rounds, each workgroup holding its
 * slab in registers from its loads to its stores, the same per-thread
 * statistics (they wait for each round's loads) and barriers -- but no
 * exchange between workgroups and no normalisation.  Its time is the
 * ceiling of that pattern.  Applies where the fused kernel does (hw a
 * multiple of 4, x and y 16-byte aligned, at most 64 slabs per channel and
 * 64 rounds); other shapes are rejected.  No counterpart in the reference;
 * used only to price a kernel's access pattern.
 */
int hipo_hold_copy_f32(const float* x, float* y, int64_t n, int64_t c, int64_t hw,
                       hipStream_t stream);


/*
 * GELU(tanh) of a contiguous tensor of n elements, element by element:
 *   bf16: y = the correctly rounded bf16 of 0.5 x (1 + tanh(sqrt(2/pi)
 *         (x + 0.044715 x^3))) for every bf16 x (no intermediate rounding);
 *   fp32: the same function as x / (1 + e^(-2u)), u = sqrt(2/pi) (x +
 *         0.044715 x^3), with an extended-precision exp and an IEEE division
 *         (a few fp32 ulps from the exact value; no cancellation).
 * x and y are 16-byte aligned and do not overlap.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/pointwise_2d969ac9ad59/oracle.py:44-62 (_tanh_gelu_kernel,
 * same file :12-26), whose view-reshape wrapper stays in Python.
 */
int hipo_gelu_tanh_bf16(const uint16_t* x, uint16_t* y, int64_t n, hipStream_t stream);
int hipo_gelu_tanh_f32(const float* x, float* y, int64_t n, hipStream_t stream);

/*
 * Batched transpose of the last two dimensions, bit for bit:
 *   y[b, c, r] = x[b, r, c],  x [batch, rows, cols], y [batch, cols, rows],
 * both contiguous, elements of elem_size bytes (2 or 4), x and y distinct.
 * permute(0, 1, 3, 2) + clone of a contiguous 4-D tensor is the case
 * batch = d0 * d1.  Replaces the Triton body of oracle_forward in
 * repros/canonical/pointwise_021e90d9c17d/oracle.py:55-80
 * (_visformer_attention_to_image_kernel, same file :23).
 */
int hipo_transpose_last2(const void* x, void* y, int64_t batch, int64_t rows,
                         int64_t cols, int elem_size, hipStream_t stream);

/*
 * bf16 row mean with an optional ReLU (relu != 0; NaN propagates):
 *   out[r] = bf16(sum_j act(x[r, j]) / cols), fp32 sum, one rounding.
 * x is contiguous [rows, cols] (cols >= 1); out is [rows].  The NCHW
 * spatial mean relu(x).mean([-1, -2]) is the case rows = N * C, cols = H * W.
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/mean_b402ee209d0b/oracle.py:53-80
 * (_relu_spatial_mean_kernel, same file :23-50).
 */
int hipo_row_mean_bf16(const uint16_t* x, uint16_t* out, int64_t rows, int64_t cols,
                       int relu, hipStream_t stream);

/* Workspace bytes of hipo_gelu_erf_bwd_colsum_bf16 (0: empty shape). */
size_t hipo_gelu_erf_bwd_colsum_workspace_bytes(int64_t rows, int64_t cols);

/*
 * GELU(erf) backward with the column sum of its output (a bias gradient):
 *   y[r, c]   = bf16(grad[r, c] * d(x[r, c])),
 *               d(t) = Phi(t) + t phi(t), the derivative of t Phi(t), taken
 *               as the correctly rounded fp32 value for each bf16 t (one
 *               fp32 product, one rounding; inf and NaN t give NaN);
 *   colsum[c] = bf16(sum_r y[r, c]) stored as fp32 (fp32 sums of the bf16 y,
 *               in a fixed order for a given shape).
 * grad, x, y are contiguous [rows, cols] bf16, 16-byte aligned, cols a
 * multiple of 8; colsum is [cols] fp32.  `workspace` holds fp64 partial sums:
 * at least hipo_gelu_erf_bwd_colsum_workspace_bytes(rows, cols) bytes,
 * 16-byte aligned, no initialisation needed; NULL when that is 0 (up to 256
 * rows, a single launch; rows == 0 sets colsum to zero).
 * Replaces the Triton body of oracle_forward in
 * repros/canonical/sum_139a3020e8bf/oracle.py:101-152
 * (_materialize_partial_kernel :13, _final_sum_kernel :62) for the graph of
 * repros/canonical/sum_139a3020e8bf/repro.py:24-48.
 */
int hipo_gelu_erf_bwd_colsum_bf16(const uint16_t* grad, const uint16_t* x, uint16_t* y,
                                  float* colsum, int64_t rows, int64_t cols,
                                  void* workspace, size_t workspace_bytes,
                                  hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* HIP_ORACLES_H_ */
