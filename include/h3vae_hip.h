/*
 * h3vae_hip.h -- C ABI of libh3vae_hip.so, the MI355X (gfx950) kernels of the
 * H3 video-VAE INT8 hot path.
 *
 * Conventions shared by every entry point:
 *   - plain device pointers and sizes; fp16 tensors are passed as uint16_t
 *     bit patterns, int8 as int8_t, scales as float;
 *   - `stream` is a hipStream_t (NULL = the default stream); work is queued
 *     asynchronously, nothing synchronises the host;
 *   - no entry point allocates memory: scratch space is passed in by the caller;
 *   - return 0 on success or an H3V_E* code; h3v_last_error() then holds the
 *     message for the calling thread.  Shape, alignment and contract checks
 *     run before anything is queued.
 *
 * Each declaration names the reference interface it replaces
 * (fishelegs/ComfyUI-H3VAE-PyOpt, file:line).
 */
#ifndef H3VAE_HIP_H
#define H3VAE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define H3V_ABI_VERSION 5

#define H3V_OK 0
#define H3V_EINVAL 1   /* shape / dtype / alignment / contract violation */
#define H3V_ELAUNCH 2  /* the HIP runtime rejected a launch */

/* The same typedef as the HIP runtime's own; repeating it is valid C11 and C++. */
typedef struct ihipStream_t* hipStream_t;

/* ABI version of the loaded library (H3V_ABI_VERSION). */
int h3v_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* h3v_last_error(void);

/* ---- row quantization (comfy-kitchen 0.2.34 contract) -------------------
 * Replaces the reference's restated CK row quantizer
 * (opt/int8_ffn_up_fused.py:91-104 `quantize_act`, and the dynamic
 * activation quant inside CK int8_linear, opt/kitchen_int8.py:20-37).
 * x: fp16 [rows, cols]; q: int8 [rows, cols]; scale: fp32 [rows].
 *   s = max(amax * fp32(1/127), 1e-30); d = fp16(s);
 *   q = clamp(rint(fp16(x / d)), -128, 127), NaN -> -128.              */
int h3v_row_quant(const uint16_t* x, int64_t rows, int64_t cols, int8_t* q, float* scale,
                  hipStream_t stream);

/* SiLU(gate) * up then row quantization of x: fp16 [rows, 2*cols] = [gate | up].
 * Replaces opt/int8_swiglu_fused.py:22-38 (`quant`) / :52-65 (`quantize_swiglu`). */
int h3v_swiglu_row_quant(const uint16_t* x, int64_t rows, int64_t cols, int8_t* q, float* scale,
                         hipStream_t stream);

/* Device self-test of the fast quotients the quantizers use instead of IEEE
 * division (no counterpart in the reference; it backs the bit-exactness claim).
 * counts: 3 uint32 of device memory, overwritten with the number of mismatches
 * against IEEE division: [0] fp32 quotients and [1] int8 codes (scalar and
 * packed-fp16 code chains) over every fp16 numerator (infinities excluded) and
 * every finite positive fp16 divisor, [2] SiLU over every fp16 argument.  All
 * three are zero on a correct build. */
int h3v_selftest_fast_div(uint32_t* counts, hipStream_t stream);

/* ---- encoder suffix / FP16 mode: GroupNorm + SiLU + pad producer, fp16 out ----
 * Replaces opt/encoder_fused_batched_norm.py:15-66 (`batched_temporal_norm_pack`,
 * its _partial/_merge/_normalize_pack_batched kernels) and, for batch one,
 * opt/encoder_fused_temporal_norm.py:83-99 / opt/encoder_fused_norm_bias.py:14-39.
 * x: fp16 NDHWC [batch * d, h, w, c] (batch and time adjacent), c in
 * {128, 256, 512, 1024}; optional pre_bias [c] (v = fp16(v + pre_bias) first).
 * Per-frame GroupNorm(32) statistics of every (batch item, frame) -> stats fp32
 * [batch * d, 32, 2] (mean, rstd); y: fp16 NDHWC [batch, d+2, h+2, w+2, c] =
 * fp16(SiLU(fp16(((v - mean) * rstd) * gamma + beta))), two zero frames and a
 * reflect border of 1 per batch item.  workspace: fp32
 * [h3v_gn_norm_pack_f16_workspace_floats(batch, c, d, h, w)] (chunk partials). */
int64_t h3v_gn_norm_pack_f16_workspace_floats(int batch, int c, int d, int h, int w);
int h3v_gn_norm_pack_f16(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma, const uint16_t* beta,
                         float eps, int batch, int c, int d, int h, int w, uint16_t* y, float* stats, float* workspace,
                         hipStream_t stream);

/* FP16 valid convolution of a padded input (the model's FP16 encoder convs:
 * after the producers above, opt/encoder_fused_batched_norm.py:83,94,96 and
 * opt/encoder_fused_norm_bias.py:135,139, and the downsample convs,
 * opt/encoder_fused_residual_pack.py:85 and opt/encoder_internal_padding.py:34;
 * F.conv3d on cuDNN in the reference).  x: fp16 NDHWC
 * [batch, d, h, wd, cin] (already padded); w: fp16 [cout, kd*kh*kw*cin] packed
 * (kd, kh, kw, c) with c fastest; bias: fp16 [cout] (nullable); out: fp16
 * NDHWC [batch, do, ho, wo, cout] with do = (d - kd) / sd + 1 (likewise ho,
 * wo) = fp16(sum fp32 + bias), fp32 accumulation on v_mfma_f32_32x32x16_f16;
 * residual (nullable, same layout as out, not aliasing it) adds the residual
 * block's closing `shortcut(x) + h` as fp16(fp32(residual) + fp32(out)).
 * causal_skip (kd == 3, sd == 1 only): output frames 0 and 1 of each batch
 * item skip the depth taps that read the two leading zero frames.  Requires
 * cin % 32 == 0 and 16-byte aligned x and w.  Stride-1 3x3x3 convs with
 * cout % 128 == 0, an output width of 32, 64, 128 or 256 and an output height
 * that is a multiple of 512 / width run with the input window in LDS; others
 * as an implicit GEMM. */
int h3v_conv3d_f16(const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,
                   uint16_t* out, int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw, int sd,
                   int sh, int sw, int causal_skip, hipStream_t stream);

/* The same convolution with a caller workspace for a split reduction (the
 * same model call sites as h3v_conv3d_f16).  When the implicit GEMM would
 * leave most CUs idle (fewer tiles than half a round of the 256 CUs) and K is
 * long, the reduction is split S ways: S workgroups per tile write fp32
 * partial sums to workspace [S, M, cout], and a second kernel adds them in
 * split order and applies the same epilogue (fp16(sum + bias), then the
 * residual).  The sums' order differs from h3v_conv3d_f16's, the values stay
 * within the same float64 bound.  workspace_floats must be at least
 * h3v_conv3d_f16_workspace_floats() of the same geometry (16-byte aligned);
 * a geometry that does not split ignores the workspace (it may be null). */
int h3v_conv3d_f16_ws(const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,
                      uint16_t* out, int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw,
                      int sd, int sh, int sw, int causal_skip, float* workspace, int64_t workspace_floats,
                      hipStream_t stream);

/* fp32 workspace floats h3v_conv3d_f16_ws needs for this geometry: 0 when it
 * does not split, -1 for an invalid geometry (h3v_last_error says why). */
int64_t h3v_conv3d_f16_workspace_floats(int batch, int cin, int d, int h, int wd, int cout, int kd, int kh, int kw,
                                        int sd, int sh, int sw);

/* h3v_conv3d_f16 (batch one, no residual, 128 output channels, an output
 * frame of a multiple of 256 pixels) that also writes the GroupNorm(32)
 * partial statistics of its output for the INT8 producer that normalises it
 * next: `workspace` (h3v_gn_norm_pack_workspace_floats of the output's
 * [d, h, w], 16-byte aligned) receives, per 256-pixel chunk of a frame, the
 * group averages and M2 and the channel max / min, in the order of that
 * producer's own statistics pass; hand it to h3v_gn_norm_pack_i8_partials
 * with chunk = 256 and no pre_bias.  Replaces the `_partial` launch of
 * _norm_statistics (opt/encoder_int8_norm.py:16-50) that follows conv_in and
 * the stage-0 downsample (the model's convs at opt/encoder_internal_padding.py:34). */
int h3v_conv3d_f16_gn(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* out, int cin, int d,
                      int h, int wd, int cout, int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip,
                      float* workspace, hipStream_t stream);

/* ---- decoder attention (head_dim 64) --------------------------------------
 * Replaces the model's `perform_attention` (flash attention) called from
 * opt/decoder_fused_qk_rope.py:66-74 (`FusedQKAttention.forward`) between the
 * fused QK-RoPE and the attention-out linear.  Non-causal, unmasked:
 *   o[b, t, h, :] = sum_s softmax_s(scale * q[b, t, h, :] . k[b, s, h, :]) v[b, s, h, :]
 * q, k, v, o: fp16 [batch, tokens, heads, 64] with the given token and head
 * strides in elements (multiples of 8; the 64 dims contiguous; batch stride =
 * tokens * token stride), so q/k can be the QK-RoPE outputs and v the strided
 * slice of the QKV projection.  fp32 softmax and accumulation, fp16 output. */
int h3v_attention_d64(const uint16_t* q, int64_t q_token_stride, int64_t q_head_stride, const uint16_t* k,
                      int64_t k_token_stride, int64_t k_head_stride, const uint16_t* v, int64_t v_token_stride,
                      int64_t v_head_stride, uint16_t* o, int64_t o_token_stride, int64_t o_head_stride,
                      int64_t batch, int64_t tokens, int64_t heads, float scale, hipStream_t stream);

/* ---- decoder edge: pixel finalisation ------------------------------------
 * Replaces opt/fp16_finalize.py:24-54 (`finalize_pixels`, its Triton kernel).
 * x: decoded pixels [batch, 3, frames, height, width], fp16 (x_is_f16 = 1,
 * uint16_t bit patterns) or fp32 (x_is_f16 = 0), element strides in
 * strides[0..4] (host memory, any layout); std, mean: fp32 [3] device
 * memory; out: contiguous fp32 [batch, 3, frames, height, width].
 *   v = fp32(x) * std[c] + mean[c]   (two roundings, no FMA)
 *   out = v < 0 ? 0 : (v > 1 ? 1 : v)   (NaN and an in-range -0 kept)       */
int h3v_finalize_pixels(const void* x, int x_is_f16, int64_t batch, int64_t frames, int64_t height, int64_t width,
                        const int64_t* strides, const float* std, const float* mean, float* out, hipStream_t stream);

/* MFMA ceiling microbenchmark (no counterpart in the reference; it measures the
 * ceiling the INT8 kernels are judged against).  `blocks` workgroups of 8 waves
 * (launch one per CU) each run iters x 32 back-to-back v_mfma_i32_32x32x32_i8
 * per wave on register-resident fragments read from a[0:a_bytes) and
 * b[0:b_bytes) (16-byte aligned int8 data, e.g. a workload's quantized
 * activations and weights: the sustained clock depends on the data).
 * sink: int32 [blocks * 512] (written, keeps the MFMAs live); clocks: int64
 * [2 * blocks], per workgroup {shader-clock ticks, 100 MHz reference ticks}
 * over the timed loop, so clock = ticks[0] / ticks[1] * 100 MHz.
 * h3v_probe_mfma_ops_per_block(iters) = INT8 ops one workgroup performs. */
int h3v_probe_mfma_rate(const int8_t* a, int64_t a_bytes, const int8_t* b, int64_t b_bytes, int blocks,
                        int iters, int32_t* sink, int64_t* clocks, hipStream_t stream);
int64_t h3v_probe_mfma_ops_per_block(int iters);

/* ---- INT8 GEMMs (int32 accumulation on MFMA) ---------------------------
 * acc[m, n] = sum_k a[m, k] * w[n, k]; a: int8 [m, k], w: int8 [n, k], both
 * row-major.  Dequant epilogue:
 *   out = fp16(bias ? fma(fp32(acc) * a_scale[m], w_scale[n], fp32(bias[n]))
 *                   : (fp32(acc) * a_scale[m]) * w_scale[n])
 * Replaces the CK CUTLASS GEMM behind prequantized_linear
 * (opt/int8_swiglu_fused.py:78-107, cutlass_int8_dequant). */
int h3v_gemm_i8_dequant(const int8_t* a, const float* a_scale, const int8_t* w, const float* w_scale,
                        const uint16_t* bias, uint16_t* out, int64_t m, int64_t n, int64_t k,
                        hipStream_t stream);

/* FFN-up GEMM with the paired SwiGLU epilogue.  w: int8 [2n, k] with gate rows
 * 0..n-1 and up rows n..2n-1; w_scale, bias: [2n].  act: fp16 [m, n] =
 *   fp16(silu(g) * u), g, u = fp32(fp16(dequant(acc of gate / up row))).
 * Replaces opt/int8_ffn_up_fused.py:50-89 (`up_swiglu`). */
int h3v_gemm_i8_swiglu(const int8_t* a, const float* a_scale, const int8_t* w, const float* w_scale,
                       const uint16_t* bias, uint16_t* act, int64_t m, int64_t n, int64_t k,
                       hipStream_t stream);

/* Raw int32 accumulators of the same GEMM (exactness checks; tl.dot with
 * out_dtype=int32 in opt/int8_ffn_up_fused.py:68-72). acc: int32 [m, n]. */
int h3v_gemm_i8_i32(const int8_t* a, const int8_t* w, int32_t* acc, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream);

/* ---- encoder convolution -----------------------------------------------
 * Valid conv3d as implicit GEMM.  qx: int8 NDHWC [batch, d, h, w, cin] (already
 * padded); qw: int8 [cout, kd*kh*kw*cin] with k = (kd, kh, kw, c), c fastest;
 * x_scale: one fp32 on the device; w_scale: fp32 [cout]; bias: fp16 [cout] or
 * NULL; out: fp16 NDHWC [batch, do, ho, wo, cout], do = (d-kd)/sd+1 etc.
 * causal_skip != 0 promises that input frames 0 and 1 are zero (the fused
 * producer's causal planes); taps that only read them are skipped (exact).
 * Replaces _conv3d_from_quantized + implicit_conv3d_kernel
 * (opt/encoder_int8.py:509-588, opt/encoder_int8_pipeline.py:15-119). */
int h3v_conv3d_i8(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                  const uint16_t* bias, uint16_t* out, int batch, int cin, int d, int h, int w, int cout,
                  int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip, hipStream_t stream);

/* The same conv with the residual block's closing add fused into the epilogue:
 * out = fp16(fp32(residual) + fp32(y)) with y the fp16 output above, i.e. the
 * `shortcut(x) + h` (or `x + h`) of opt/encoder_fused_norm_bias.py:141
 * (BiasFusedResidualBlock.forward) in one pass instead of a separate add kernel;
 * bit-identical to the conv followed by torch's fp16 add.  residual: fp16 NDHWC
 * [batch, do, ho, wo, cout], not aliasing out. */
int h3v_conv3d_i8_residual(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                           const uint16_t* bias, const uint16_t* residual, uint16_t* out, int batch, int cin, int d,
                           int h, int w, int cout, int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip,
                           hipStream_t stream);

/* The last convolution of an encoder stage with its output written straight
 * into the padded input of the stage's causal stride-2 downsample, so that no
 * pack kernel re-reads it.  Replaces the conv + pack pairs of
 * opt/encoder_fused_residual_pack.py:12-46 (stage 1: the second conv without
 * bias, then residual_downsample_pack; border 0, 1, 0, 1) and, for the stage-0
 * downsample, the block's residual conv followed by the zero frames and
 * reflect padding of opt/encoder_internal_padding.py:27-36 (border 1, 1, 1, 1).
 * A stride-1 3x3x3 conv (kd = kh = kw = 3): y = the fp16 output of
 * h3v_conv3d_i8 (bias nullable); with residual (fp16 NDHWC [batch, do, ho, wo,
 * cout]) v = fp16(fp32(residual) + fp32(y)), or with residual_bias (fp16
 * [cout], the pack's bias) v = fp16(fp32(residual) + (fp32(y) +
 * fp32(residual_bias))), one rounding.  out: fp16 NDHWC [batch, do + front,
 * ho + top + bottom, wo + left + right, cout] with a reflect border of 0 or 1
 * per side: out[b, front + t, top + i, left + j] = v[b, t, i, j]; row 1 is
 * repeated as row 0 (top), row ho - 2 as row ho + top (bottom), likewise the
 * columns; frames below `front` are not written (the caller zeroes them).
 * Requires Cin % 64 == 0, Cout % 128 == 0, wo in {32, 64, 128, 256}, ho a
 * multiple of 512 / wo and >= 2, 16-byte aligned out / residual /
 * residual_bias, front in [0, 16]. */
int h3v_conv3d_i8_residual_padded(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                                  const uint16_t* bias, const uint16_t* residual, const uint16_t* residual_bias,
                                  uint16_t* out, int batch, int cin, int d, int h, int w, int cout, int causal_skip,
                                  int front, int top, int bottom, int left, int right, hipStream_t stream);

/* h3v_conv3d_i8 / h3v_conv3d_i8_residual (batch one, stride-1 3x3x3) that also
 * writes the GroupNorm(32) statistics the next INT8 producer needs of its
 * output, so that producer skips its own statistics pass over it.  Replaces,
 * for the convolution that feeds a norm, the `_partial` / `_partial_bias`
 * launches of _norm_statistics (opt/encoder_int8_norm.py:16-50, kernels of
 * opt/encoder_fused_temporal_norm.py and opt/encoder_fused_norm_bias.py:14-39)
 * that follow _conv3d_from_quantized (opt/encoder_int8.py:509).
 * out (and residual, nullable): fp16 NDHWC [1, do, ho, wo, cout] as in those
 * entry points; gn_bias: fp16 [cout] or NULL, the next producer's pre_bias
 * (statistics of fp16(out + gn_bias)).  workspace: the next producer's
 * workspace (h3v_gn_norm_pack_workspace_floats(do, ho, wo) floats), filled
 * with the partial statistics of every 8-row x 64-column output tile (512
 * pixels: per tile and group the average and M2, per tile and channel the
 * fp16 max and min); hand it to h3v_gn_norm_pack_i8_partials with the same
 * pre_bias.  Requires cin % 128 == 0, cout 128 or 256, wo 128 or 256, ho a
 * multiple of 8, 16-byte aligned out, residual, gn_bias and workspace. */
int h3v_conv3d_i8_gn(const int8_t* qx, const float* x_scale, const int8_t* qw, const float* w_scale,
                     const uint16_t* bias, const uint16_t* residual, uint16_t* out, int cin, int d, int h, int w,
                     int cout, int causal_skip, const uint16_t* gn_bias, float* workspace, hipStream_t stream);

/* Raw int32 accumulators of the same convolution (exactness checks). */
int h3v_conv3d_i8_i32(const int8_t* qx, const int8_t* qw, int32_t* acc, int batch, int cin, int d, int h,
                      int w, int cout, int kd, int kh, int kw, int sd, int sh, int sw, int causal_skip,
                      hipStream_t stream);

/* Per-tensor dynamic activation quant of a contiguous fp16 tensor of n
 * elements: scale = amax * fp32(1/127) (0 -> 1), q = clamp(half-away(x/scale),
 * +-127).  scratch: scratch_words 32-bit words of device scratch (partial
 * maxima; nothing needs clearing between calls), at least
 * h3v_tensor_quant_scratch_words(); a shorter one is rejected (H3V_EINVAL).
 * Replaces quantize_activation_tensor (opt/encoder_int8.py:384-426). */
int64_t h3v_tensor_quant_scratch_words(void);
int h3v_tensor_quant_i8(const uint16_t* x, int64_t n, int8_t* q, float* scale, uint32_t* scratch,
                        int64_t scratch_words, hipStream_t stream);

/* Float count of the workspace h3v_gn_norm_pack_i8 needs for a [d, h, w] input. */
int64_t h3v_gn_norm_pack_workspace_floats(int d, int h, int w);

/* Fused GroupNorm(32) / SiLU / causal + reflect pad / INT8 producer.
 * x: fp16 NDHWC [d, h, w, c] (batch one, c in {128, 256}); pre_bias: fp16 [c]
 * or NULL (v = fp16(v + pre_bias) first); gamma, beta: fp16 [c].
 * q: int8 NDHWC [d+2, h+2, w+2, c]; scale: one fp32; stats: fp32 [d, 32, 2]
 * (mean, rstd); workspace: h3v_gn_norm_pack_workspace_floats() floats;
 * amax_scratch: one uint32.
 * Replaces quantized_temporal_norm_pad (opt/encoder_int8_norm.py:77-110)
 * with _partial/_partial_bias/_merge and recompute_pack. */
int h3v_gn_norm_pack_i8(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma, const uint16_t* beta,
                        float eps, int c, int d, int h, int w, int8_t* q, float* scale, float* stats,
                        float* workspace, uint32_t* amax_scratch, hipStream_t stream);

/* h3v_gn_norm_pack_i8 on an input whose producing conv wrote its GroupNorm
 * partial statistics into `workspace` (summed over x + pre_bias with the same
 * pre_bias); the statistics pass is skipped and the chunks merge in order.
 * chunk = 512: the 512-pixel tiles of h3v_conv3d_i8_gn (h * w a multiple of
 * 512, h >= 8; 8-row bands of 64-column blocks), the same outputs as
 * h3v_gn_norm_pack_i8 up to the summation order of the statistics;
 * chunk = 256: the 256-pixel chunks of h3v_conv3d_f16_gn (h * w a multiple
 * of 256), written in the statistics pass's own order, so the outputs are
 * bit-identical to h3v_gn_norm_pack_i8's.  Replaces
 * quantized_temporal_norm_pad (opt/encoder_int8_norm.py:77-110) after the
 * fused conv. */
int h3v_gn_norm_pack_i8_partials(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma,
                                 const uint16_t* beta, float eps, int c, int d, int h, int w, int chunk, int8_t* q,
                                 float* scale, float* stats, float* workspace, uint32_t* amax_scratch,
                                 hipStream_t stream);

/* h3v_gn_norm_pack_i8 without a workspace argument and without allocating:
 * no counterpart in the reference.  It is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The workspace and the absmax word live in a static
 * device array of the library, one per GPU, 8 MiB + 256 bytes, held until the
 * process ends; a call whose h3v_gn_norm_pack_workspace_floats(d, h, w)
 * exceeds 2097152 floats is rejected with H3V_EINVAL (256 x 256 frames: up to
 * d = 25).  The array of the current device is used, so `stream` must belong
 * to it.  Every call on one GPU shares that array; calls that overlap on one
 * GPU (two streams or threads) race.  Same inputs, outputs and results as
 * h3v_gn_norm_pack_i8. */
int h3v_gn_norm_pack_i8_noalloc(const uint16_t* x, const uint16_t* pre_bias, const uint16_t* gamma,
                                const uint16_t* beta, float eps, int c, int d, int h, int w, int8_t* q, float* scale,
                                float* stats, hipStream_t stream);

/* ---- decoder row producers (row width k in {1024, 2048, 4096}) ---------
 * norm1: raw = fma(o, g, h); h_out = fp16(raw) (h_out may equal h: in place);
 * ss = published W16 tree of raw^2; inv = 1/sqrt(ss/k + eps);
 * n = fp16((fp32(h_out) * inv) * w); (q, scale) = row quantization of n.
 * Replaces residual_norm_quant via _produce_norm1 (opt/int8_norm1_quant.py:113-123). */
int h3v_residual_norm1_quant(const uint16_t* h, const uint16_t* o, const uint16_t* g, const uint16_t* w, float eps,
                             int64_t m, int64_t k, uint16_t* h_out, int8_t* q, float* scale, hipStream_t stream);

/* norm2: as norm1 with the plain tree of rounded squares.
 * Replaces residual_quant (opt/int8_norm_quant.py:22-69). */
int h3v_residual_rms_quant(const uint16_t* x, const uint16_t* a, const uint16_t* g, const uint16_t* w, float eps,
                           int64_t m, int64_t k, uint16_t* h_out, int8_t* q, float* scale, hipStream_t stream);

/* Block-0 RMSNorm: out = fp16((x * inv) * gamma), W16 tree of x^2.
 * Replaces rms_fp16_x2_w16 (opt/decoder_block0_norm.py:39-95). */
int h3v_rms_fp16(const uint16_t* x, const uint16_t* gamma, float eps, int64_t m, int64_t k, uint16_t* out,
                 hipStream_t stream);

/* Final residual + LayerNorm: raw = fma(o, gate, h);
 * out = fp16(fma((raw - mean) * inv, gamma, beta)).
 * Replaces final_residual_ln_w8 (opt/decoder_final_norm.py:35-86). */
int h3v_residual_layernorm(const uint16_t* h, const uint16_t* o, const uint16_t* gate, const uint16_t* gamma,
                           const uint16_t* beta, float eps, int64_t m, int64_t k, uint16_t* out,
                           hipStream_t stream);

/* ---- attention input ---------------------------------------------------
 * QK RMSNorm (no affine) + rotate-half RoPE on the first rot_dim dims.
 * qkv: fp16 [tokens, heads, 3*head_dim] (per head [q | k | v]);
 * cosv, sinv: fp16 [tokens, rot_dim]; q, k: fp16 [tokens, heads, head_dim].
 * head_dim must be 64 and rot_dim 48.
 * Replaces qk_rope / _qk_rope (opt/decoder_fused_qk_rope.py:12-54). */
int h3v_qk_rope(const uint16_t* qkv, const uint16_t* cosv, const uint16_t* sinv, int64_t tokens, int heads,
                int head_dim, int rot_dim, float eps, uint16_t* q, uint16_t* k, hipStream_t stream);

/* Residual + bias pack ahead of the stride-2 downsample conv of the last encoder prefix block.
 * x, residual: fp16 NDHWC [d, h, w, c] (batch one); bias: fp16 [c];
 * out: fp16 NDHWC [d+2, h+1, w+1, c] = two leading zero frames, then
 * fp16(residual + (x + bias)) (fp32 adds, one rounding) with one reflected row/column at the
 * bottom/right (index h -> h-2, w -> w-2).  c % 8 == 0, h, w >= 2, 16-byte aligned buffers.
 * Replaces residual_downsample_pack / _residual_pack (opt/encoder_fused_residual_pack.py:12-55). */
int h3v_residual_downsample_pack(const uint16_t* x, const uint16_t* residual, const uint16_t* bias, uint16_t* out,
                                 int c, int d, int h, int w, hipStream_t stream);

/* Causal/reflect pack ahead of an FP16 convolution whose input the model pads
 * itself: F.pad(reflect) + the causal zero frames of CausalConv3d, as used by
 * opt/encoder_internal_padding.py:27-35 (`ImplicitTemporalPadConv3d`, where
 * the zero frames are the conv's temporal padding) and the model's downsample
 * convs.  x: fp16 NDHWC [batch, d, h, w, c]; out: fp16 NDHWC
 * [batch, d + front, h + top + bottom, w + left + right, c]: `front` zero frames
 * per item, then x with the spatial border reflected (-p -> p, h-1+p -> h-1-p).
 * c % 8 == 0, each reflect pad smaller than its dimension, 16-byte aligned. */
int h3v_causal_reflect_pack(const uint16_t* x, uint16_t* out, int batch, int c, int d, int h, int w, int front,
                            int top, int bottom, int left, int right, hipStream_t stream);

/* Tap-folded pack for the encoder's conv_in (the model's CausalConv3d with 3
 * input channels, run as F.conv3d by the reference: it is not replaced there).
 * x: fp16 NDHWC [batch, d, h, w, c]; out: fp16 NDHWC [batch, d + front, h, w, cf]
 * with out[.., t, i, j, (kh*3 + kw)*c + ch] = x[.., t - front, r(i + kh - 1),
 * r(j + kw - 1), ch] (r: reflect) for t >= front and zero otherwise, channels
 * 9c .. cf-1 zero.  The 3x3x3 conv becomes a 3x1x1 conv over cf channels
 * (h3v_conv3d_f16).  cf == 32, c in 1..3, h, w >= 2, 16-byte aligned out. */
int h3v_tap_fold_pack(const uint16_t* x, uint16_t* out, int batch, int c, int d, int h, int w, int front, int cf,
                      hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* H3VAE_HIP_H */
