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
 * Replaces: mixed_linear (mixed_precision/triton_linear.py:221-269).
 */
int mpk_linear(const void* x, int x_dtype, const void* w, const void* b, void* y, int y_dtype, int gelu,
               int64_t m, int32_t n, int32_t k, int variant, void* stream);
int mpk_linear_auto_variant(int64_t m, int32_t n, int32_t k);

/*
 * Projection + residual + LayerNorm:
 *   residual_out = fp16(x) * w^T + b + residual          (FP32)
 *   normalized_out = LayerNorm(residual_out) * gamma + beta
 * x: [m, d] in x_dtype; w: [d, d] FP16; b: [d] FP16; residual, residual_out:
 * [m, d] FP32; gamma, beta: [d] FP32.  d in {32, 64, 128, 256, 512}.
 * Replaces: mixed_linear_add_layer_norm (mixed_precision/triton_linear.py:272-324).
 */
int mpk_linear_residual_layernorm(const void* x, int x_dtype, const void* w, const void* b,
                                  const float* residual, const float* gamma, const float* beta,
                                  float* residual_out, void* normalized_out, int normalized_dtype,
                                  int64_t m, int32_t d, float eps, int variant, void* stream);
int mpk_linear_residual_layernorm_auto_variant(int64_t m, int32_t d);

/*
 * Whole FFN + residual + LayerNorm, hidden activation kept on chip:
 *   h = GELU_erf(fp16(x) * w_in^T + b_in)                 (FP32, then FP16)
 *   residual_out = h * w_out^T + b_out + residual          (FP32)
 *   normalized_out = LayerNorm(residual_out) * gamma + beta
 * x: [m, d]; w_in: [f, d] FP16; b_in: [f] FP16; w_out: [d, f] FP16;
 * b_out: [d] FP16.  d in {32, 64, 128, 256, 512}; f % 32 == 0.
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
 * head_dim in {16, 32, 64, 128}.
 * Replaces: fp16_causal_attention (custom_kernel/triton_attention.py:341-390)
 *           and causal_attention (custom_kernel/triton_attention.py:320-338).
 */
int mpk_causal_attention(const void* q, const void* k, const void* v, void* o, int io_dtype, int out_dtype,
                         const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* o_strides, int32_t batch, int32_t heads, int32_t seq_len,
                         int32_t head_dim, float scale, int causal, const uint8_t* key_valid, int variant,
                         void* stream);
int mpk_attention_auto_variant(int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim);

#ifdef __cplusplus
}
#endif

#endif /* MPK_H_ */
