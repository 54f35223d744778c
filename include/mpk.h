/*
 * mpk.h - C ABI of libmpk.so, the gfx950 (MI355X) kernels behind the
 * mixed-precision causal-Transformer forward.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and a HIP stream passed as
 *     `void*` (a hipStream_t; NULL = the default stream);
 *   - is asynchronous on that stream, allocates nothing, frees nothing and
 *     performs no host synchronisation (safe under HIP graph capture);
 *   - returns 0 on success, MPK_EINVAL / MPK_EUNSUPPORTED / MPK_EALIGN for
 *     rejected arguments (checked on the host before any launch), or a
 *     hipError_t value from the launch; mpk_status_string() names it.
 * Buffers must be 16-byte aligned and row-contiguous unless stated otherwise.
 * dtype codes: MPK_F32 = 0 (float), MPK_F16 = 1 (IEEE binary16).
 * FP16 tensors are passed as `const void*` holding binary16 bits.
 * `variant` selects a kernel tile configuration; 0 = the built-in dispatch
 * table (see the *_auto_variant queries).
 */
#ifndef MPK_H_
#define MPK_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MPK_F32 0
#define MPK_F16 1

#define MPK_OK 0
#define MPK_EINVAL 1001
#define MPK_EUNSUPPORTED 1002
#define MPK_EALIGN 1003

int mpk_version(void);
const char* mpk_status_string(int status);
int mpk_device_synchronize(void);

/*
 * Residual add + LayerNorm with FP32 statistics, or a plain LayerNorm.
 *   r = x + update (update may be NULL: r = x, residual_out unused)
 *   normalized_out = (r - mean) * rsqrt(var + eps) * gamma + beta   (biased var)
 * x, update, residual_out: [rows, d] FP32; gamma, beta: [d] FP32;
 * normalized_out: [rows, d] in normalized_dtype. d % 4 == 0, d <= 2048.
 * Replaces: fused_add_layer_norm (torch_transformer_benchmark.py:72-103),
 *           mixed_add_layer_norm (mixed_precision/triton_linear.py:381-424),
 *           the initial norm1 + cast (mixed_precision/transformer.py:484-486).
 */
int mpk_layernorm(const float* x, const float* update, const float* gamma, const float* beta,
                  float* residual_out, void* normalized_out, int normalized_dtype, int64_t rows,
                  int32_t d, float eps, void* stream);

/*
 * Projection y = act(fp16(x) * w^T + b), FP32 accumulate, act = exact-erf GELU
 * when gelu != 0.  x: [m, k] in x_dtype; w: [n, k] FP16 (nn.Linear layout);
 * b: [n] FP16; y: [m, n] in y_dtype.  n % 8 == 0, k % 8 == 0.
 * variant 0: the built-in table (mpk_linear_auto_variant); 1-9 pin a tile shape (all give
 * identical results).  8: 256x256 tiles with LDS-DMA operand staging; 9: X-stationary
 * 256-token tiles with W streamed through LDS (FP16 x, k = 128 or 256, n % 64 == 0).
 * Replaces: mixed_linear (mixed_precision/triton_linear.py:221-269).
 */
int mpk_linear(const void* x, int x_dtype, const void* w, const void* b, void* y, int y_dtype, int gelu,
               int64_t m, int32_t n, int32_t k, int variant, void* stream);

/*
 * mpk_linear without GELU, with output columns [0, q_cols) multiplied by q_scale in FP32 before
 * the output rounding: the packed QKV projection with the attention's scale * log2(e) folded
 * into q, for mpk_causal_attention_prescaled.  q_cols % 8 == 0, 0 <= q_cols <= n.
 * No single reference counterpart: the reference scales the scores instead
 * (custom_kernel/triton_attention.py:85, after mixed_linear at mixed_precision/transformer.py:88-120).
 */
int mpk_linear_qscaled(const void* x, int x_dtype, const void* w, const void* b, void* y, int y_dtype, int64_t m,
                       int32_t n, int32_t k, int32_t q_cols, float q_scale, int variant, void* stream);
int mpk_linear_auto_variant(int64_t m, int32_t n, int32_t k);

/*
 * Projection with a residual add: y = fp16(x) * w^T + b + residual  (FP32 [m, n]).
 * residual and y are FP32 [m, n]; y may be residual itself (in-place add).  n % 8 == 0, k % 8 == 0.
 * Replaces, fused: the unfused route's projection + residual add
 * (mixed_precision/transformer.py:273 out_proj, whose output is added at :501-506; :669-671 ffn_out,
 * added at :682-687); the LayerNorm of those calls follows as mpk_layernorm.
 */
int mpk_linear_residual(const void* x, int x_dtype, const void* w, const void* b, const float* residual, float* y,
                        int64_t m, int32_t n, int32_t k, int variant, void* stream);

/*
 * Projection + residual + LayerNorm:
 *   residual_out = fp16(x) * w^T + b + residual          (FP32)
 *   normalized_out = LayerNorm(residual_out) * gamma + beta
 * x: [m, d] in x_dtype; w: [d, d] FP16; b: [d] FP16; residual, residual_out:
 * [m, d] FP32; gamma, beta: [d] FP32.  d in {32, 64, 128, 256, 512}.  variant: 0 (built-in
 * choice), 1 / 2 (whole rows per wave on LDS-staged tiles), 3 (large tiles holding whole rows,
 * d 256 / 512), 4 (d 256 with FP16 x: the weights resident in LDS, independent 16-row wave
 * tiles; bit-identical to 1 and 2).
 * Replaces: mixed_linear_add_layer_norm (mixed_precision/triton_linear.py:272-324).
 */
int mpk_linear_residual_layernorm(const void* x, int x_dtype, const void* w, const void* b,
                                  const float* residual, const float* gamma, const float* beta,
                                  float* residual_out, void* normalized_out, int normalized_dtype,
                                  int64_t m, int32_t d, float eps, int variant, void* stream);
int mpk_linear_residual_layernorm_auto_variant(int64_t m, int32_t d);

/*
 * Projection with any input width + residual + LayerNorm, on GEMM tiles that hold
 * whole rows (256 x 256 for n == 256, 128 x 512 for n == 512) and whose LayerNorm
 * statistics are exchanged across waves in LDS:
 *   residual_out = fp16(x) * w^T + b + residual            (FP32)
 *   normalized_out = LayerNorm(residual_out) * gamma + beta
 * x: [m, k] in x_dtype; w: [n, k] FP16; b: [n] FP16; residual, residual_out:
 * [m, n] FP32 (residual_out may alias residual); gamma, beta: [n] FP32.
 * n in {256, 512}, k % 8 == 0.
 * Replaces, for the wide route, the reference's FFN-output projection plus its
 * residual add and the next LayerNorm (generic FFN mixed_precision/transformer.py:664-672
 * followed by mixed_add_layer_norm / fused_add_layer_norm at :674-690); with k == n it
 * is mixed_linear_add_layer_norm (mixed_precision/triton_linear.py:272-324).
 */
int mpk_linear_add_layernorm(const void* x, int x_dtype, const void* w, const void* b,
                             const float* residual, const float* gamma, const float* beta,
                             float* residual_out, void* normalized_out, int normalized_dtype,
                             int64_t m, int32_t n, int32_t k, float eps, void* stream);

/*
 * Whole FFN + residual + LayerNorm, hidden activation kept on chip:
 *   h = GELU_erf(fp16(x) * w_in^T + b_in)                 (FP32, then FP16)
 *   residual_out = h * w_out^T + b_out + residual          (FP32)
 *   normalized_out = LayerNorm(residual_out) * gamma + beta
 * x: [m, d]; w_in: [f, d] FP16; b_in: [f] FP16; w_out: [d, f] FP16;
 * b_out: [d] FP16.  d in {32, 64, 128, 256, 512}; f % 32 == 0.
 * residual_out may be NULL: then only normalized_out is stored (a last layer,
 * whose residual stream nothing reads).
 * variant: 0 = built-in choice (mpk_ffn_residual_layernorm_auto_variant),
 * 1 / 2 = one / two 16-token tiles per wave, 3 = the wide kernel (d 256,
 * f <= 8192, one wave per SIMD, FP16 x only: MPK_EUNSUPPORTED for FP32 x),
 * 4 = the role-split wide kernel (same shapes, FP16 or FP32 x; a vector wave
 * and a matrix wave per SIMD).  Variants 3 and 4 give identical results.
 * Replaces: mixed_ffn_add_layer_norm (mixed_precision/triton_linear.py:327-378).
 */
int mpk_ffn_residual_layernorm(const void* x, int x_dtype, const void* w_in, const void* b_in,
                               const void* w_out, const void* b_out, const float* residual,
                               const float* gamma, const float* beta, float* residual_out,
                               void* normalized_out, int normalized_dtype, int64_t m, int32_t d,
                               int32_t f, float eps, int variant, void* stream);
int mpk_ffn_residual_layernorm_auto_variant(int64_t m, int32_t d, int32_t f);

/*
 * Flash attention (online softmax, FP32 statistics), causal when causal != 0.
 * q, k, v: strided [batch, heads, seq_len, head_dim] views in io_dtype
 * (strides in elements: batch, head, seq, dim; dim stride must be 1);
 * o: same indexing in out_dtype.  key_valid: optional [batch, seq_len] bytes,
 * nonzero = key may be attended (NULL = all valid).  scale multiplies q.k.
 * head_dim in {8, 16, 32, 64, 128, 256}.  variant: 0 = built-in choice
 * (mpk_attention_auto_variant), 1..5 tile shapes of the 16x16-MFMA kernel,
 * 6..8 the 32x32-MFMA kernel (head_dim 32 and 64 only, else MPK_EUNSUPPORTED).
 * Replaces: fp16_causal_attention (custom_kernel/triton_attention.py:341-390)
 *           and causal_attention (custom_kernel/triton_attention.py:320-338).
 */
int mpk_causal_attention(const void* q, const void* k, const void* v, void* o, int io_dtype, int out_dtype,
                         const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* o_strides, int32_t batch, int32_t heads, int32_t seq_len,
                         int32_t head_dim, float scale, int causal, const uint8_t* key_valid, int variant,
                         void* stream);
int mpk_attention_auto_variant(int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim);

/*
 * mpk_causal_attention for FP16 q / k / v whose q already holds q * scale * log2(e), rounded to
 * FP16 once by its producer (mpk_linear_qscaled): the 32x32 kernel (head_dim 32 or 64, variant 0
 * or 6-8; variant 0 picks, at head_dim 32, 7 where its launch is large enough for the grouped
 * schedule - B*H a multiple of 64 and (B*H / 8) * ceil(S / 256) >= 1024 - and 6 otherwise) with
 * the scores already in log2 units, so no
 * per-score scaling.  out_dtype kF16 or kF32.
 * Replaces, with the scale moved into the projection: fp16_causal_attention
 * (custom_kernel/triton_attention.py:341-390).
 */
int mpk_causal_attention_prescaled(const void* q, const void* k, const void* v, void* o, int out_dtype,
                                   const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                   const int64_t* o_strides, int32_t batch, int32_t heads, int32_t seq_len,
                                   int32_t head_dim, int causal, const uint8_t* key_valid, int variant, void* stream);

/*
 * Whole-layer tail for narrow models: everything after attention up to the next
 * layer's QKV projection, with the activations kept on chip:
 *   x_out = fp16(ctx) w_o^T + b_o + x                               (FP32)
 *   n2    = LayerNorm(x_out; ln2_w, ln2_b, ln2_eps)                 (FP16 operand)
 *   x_out = fp16(GELU_erf(n2 w_in^T + b_in)) w_out^T + b_out + x_out (FP32)
 *   last == 0: out = LayerNorm(x_out; next_ln) w_qkv^T + b_qkv      (FP16 [m, 3d])
 *   last != 0: out = LayerNorm(x_out; next_ln)                      (FP32 [m, d])
 * ctx: [m, d] FP16; x, x_out: [m, d] FP32 (may not alias); w_o [d, d], w_in [f, d],
 * w_out [d, f], w_qkv [3d, d] and their biases FP16; LayerNorm parameters FP32.
 * (d, f) must satisfy mpk_layer_tail_supported.  variant: 0 = built-in choice (3 when
 * 128-row tiles would leave CUs idle, else 1), 1 = 8 waves x 16 rows per workgroup,
 * 2 = 8 waves x 32 rows (where its LDS footprint fits, else as 1), 3 = 4 waves x 16 rows.
 * Replaces, fused: mixed_linear_add_layer_norm + mixed_ffn_add_layer_norm +
 * the next layer's mixed_linear QKV call (mixed_precision/transformer.py:196-222,
 * :540-560, :88-120); no single reference function corresponds to it.
 */
int mpk_layer_tail(const void* ctx, const float* x, const void* w_o, const void* b_o, const float* ln2_w,
                   const float* ln2_b, const void* w_in, const void* b_in, const void* w_out, const void* b_out,
                   const float* next_ln_w, const float* next_ln_b, const void* w_qkv, const void* b_qkv,
                   float* x_out, void* out, int last, int64_t m, int32_t d, int32_t f, float ln2_eps,
                   float next_ln_eps, int variant, void* stream);
int mpk_layer_tail_supported(int32_t d, int32_t f);

/*
 * mpk_layer_tail with the next layer's q columns (out[:, 0:d], last == 0) multiplied by
 * q_scale in FP32 before the FP16 rounding: the next QKV for mpk_causal_attention_prescaled
 * (q_scale = scale * log2(e)).  k / v columns, x_out and the last layer's output are those of
 * mpk_layer_tail bit for bit.
 * Replaces, with the scale moved into the projection: the calls mpk_layer_tail replaces
 * (mixed_precision/transformer.py:196-222, :540-560, :88-120); no single reference function
 * corresponds to it.
 */
int mpk_layer_tail_qscaled(const void* ctx, const float* x, const void* w_o, const void* b_o, const float* ln2_w,
                           const float* ln2_b, const void* w_in, const void* b_in, const void* w_out,
                           const void* b_out, const float* next_ln_w, const float* next_ln_b, const void* w_qkv,
                           const void* b_qkv, float* x_out, void* out, int last, int64_t m, int32_t d, int32_t f,
                           float ln2_eps, float next_ln_eps, float q_scale, int variant, void* stream);

/*
 * Attention + layer tail in one kernel, for head dim 32 (or 16 at d 32 and 64): the causal
 * (or, with causal == 0, full) attention of every row over this layer's packed QKV, then
 * everything mpk_layer_tail does, the context never leaving the registers:
 *   ctx   = attention(qkv_in; heads, scale, causal)   (as mpk_causal_attention, variant 1:
 *           16x16-MFMA kernel, 64-key tiles - the same arithmetic, bit for bit)
 *   then x_out, out as mpk_layer_tail with that ctx.
 * qkv_in: [m, 3d] FP16 = [m / seq_len sequences][seq_len][q | k | v]; m % seq_len == 0 and
 * seq_len % mpk_attention_layer_tail_rows() == 0, so that every 64-row tile lies in one
 * sequence; no key mask.  out must not overlap qkv_in (other workgroups read this layer's K
 * and V while a workgroup writes the next layer's QKV): MPK_EINVAL if it does.  Shapes:
 * mpk_attention_layer_tail_supported (the layer-tail shapes whose LDS also holds the
 * attention tiles).  One launch per layer instead of mpk_causal_attention + mpk_layer_tail:
 * each 64-row workgroup computes its rows' attention itself, so it pays off for short
 * sequences of narrow models (the module route uses it at d 32 and 64 up to 128-512
 * positions by shape, measured 3-20 % faster per forward; d 128 is built but measured slower
 * than two launches).
 * Replaces, fused: fp16_causal_attention (custom_kernel/triton_attention.py:341-390) with
 * the calls mpk_layer_tail replaces; no single reference function corresponds to it.
 */
int mpk_attention_layer_tail(const void* qkv_in, const float* x, const void* w_o, const void* b_o,
                             const float* ln2_w, const float* ln2_b, const void* w_in, const void* b_in,
                             const void* w_out, const void* b_out, const float* next_ln_w, const float* next_ln_b,
                             const void* w_qkv, const void* b_qkv, float* x_out, void* out, int last, int64_t m,
                             int32_t d, int32_t f, int32_t heads, int32_t seq_len, float scale, int causal,
                             float ln2_eps, float next_ln_eps, void* stream);
int mpk_attention_layer_tail_supported(int32_t d, int32_t f, int32_t heads);
int32_t mpk_attention_layer_tail_rows(void);

/*
 * First-layer head: qkv = LayerNorm(x; ln_w, ln_b, eps) w_qkv^T + b_qkv.
 * x: [m, d] FP32; w_qkv: [3d, d] FP16; b_qkv: [3d] FP16; qkv: [m, 3d] FP16.  variant as
 * for mpk_layer_tail.
 * Replaces, fused: the initial norm1 + cast (mixed_precision/transformer.py:484-486)
 * and the first layer's QKV mixed_linear (:88-120).
 */
int mpk_layernorm_qkv(const float* x, const float* ln_w, const float* ln_b, const void* w_qkv,
                      const void* b_qkv, void* qkv, int64_t m, int32_t d, float eps, int variant, void* stream);
int mpk_layernorm_qkv_supported(int32_t d);

/*
 * mpk_layernorm_qkv with the q columns (qkv[:, 0:d]) multiplied by q_scale in FP32 before the
 * FP16 rounding (k / v columns bit for bit those of mpk_layernorm_qkv): the first layer's QKV
 * for mpk_causal_attention_prescaled.
 * Replaces, with the scale moved into the projection: the initial norm1 + cast
 * (mixed_precision/transformer.py:484-486) and the first QKV mixed_linear (:88-120).
 */
int mpk_layernorm_qkv_qscaled(const float* x, const float* ln_w, const float* ln_b, const void* w_qkv,
                              const void* b_qkv, void* qkv, int64_t m, int32_t d, float eps, float q_scale,
                              int variant, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MPK_H_ */
