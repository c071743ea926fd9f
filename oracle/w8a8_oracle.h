/*
 * CPU restatement of krea2-hrx's W8A8 transformer-product path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels and the timed CPU baseline. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Buffers follow the reference's kernel bindings exactly:
 *   f16 / bf16 values travel as uint16_t bit patterns, int8 codes as int8_t,
 *   scales as float. Rows of prepared operands are `out_stride` bytes apart and
 *   bytes past `width` in a row are never written.
 */
#ifndef K2W8_ORACLE_H
#define K2W8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scalar conversions (round to nearest, ties to even). */
uint16_t ora_bf16_from_f32(float x);
float ora_bf16_to_f32(uint16_t b);
uint16_t ora_f16_from_f32(float x);
float ora_f16_to_f32(uint16_t h);

/* The sigmoid's exponential: a fixed f32 function that the device code computes
 * bit-for-bit. */
float ora_expf(float x);

/* Element-wise helpers exposed so tests can check them in bulk. */
void ora_expf_n(const float *x, float *y, int64_t n);
void ora_sigmoid_bits_n(uint32_t first, float *y, int64_t n);
void ora_f16_from_f32_n(const float *x, uint16_t *y, int64_t n);
void ora_bf16_from_f32_n(const float *x, uint16_t *y, int64_t n);

/* Activation prepares. `threads` is the OpenMP thread count (<= 0: all). */
void ora_prepare_plain_i8(int64_t tokens, int64_t width, int64_t out_stride,
                          const uint16_t *h, int8_t *q, float *q_scale, int threads);
void ora_prepare_norm_i8(int64_t tokens, int64_t width, int64_t out_stride, float eps,
                         const uint16_t *h, const float *norm_scale, const float *mod_scale,
                         const float *mod_shift, int8_t *q, float *q_scale, int threads);
void ora_prepare_gated_i8(int64_t tokens, int64_t width, int64_t out_stride,
                          int64_t gate_stride, const uint16_t *attn, const uint16_t *gate,
                          int8_t *q, float *q_scale, int threads);

/* The canonical sum of squares of one bf16 row, exposed for tests. */
float ora_norm_sum_squares(int64_t width, const uint16_t *h_row);

/* acc[m][n] = sum_{k < k_size} a[m*k_stride+k] * w[n*k_stride+k], exact int32. */
void ora_gemm_i32(int64_t m, int64_t n, int64_t k_size, int64_t k_stride, const int8_t *a,
                  const int8_t *w, int32_t *acc, int threads);

/* Epilogues over an int32 accumulator [m][n]. */
void ora_epilogue_plain(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                        const float *a_scale, uint16_t *c_f16);
void ora_epilogue_resid(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                        const float *a_scale, const float *gate, uint16_t *x_bf16);
void ora_epilogue_swiglu(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                         const float *a_scale, uint16_t *c_f16);
/* Plain epilogue with an f16 bias added before the bf16 boundary (an
 * extension: the reference's W8A8 GEMMs carry no bias). */
void ora_epilogue_bias(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                       const float *a_scale, const uint16_t *bias_f16, uint16_t *c_f16);

/* GEMM + epilogue in one call (the CPU baseline's unit of work). */
void ora_gemm_i8(int64_t m, int64_t n, int64_t k_size, int64_t k_stride, const int8_t *a,
                 const int8_t *w, const float *w_scale, const float *a_scale, uint16_t *c_f16,
                 int threads);

/* The attention step of a block (src/session/mod.rs:714-755). */

/* kernels/rope_qknorm_f16.loom: per-head RMSNorm + rotary embedding of q and k, v copied.
 * qkv f16 [tokens][row_stride] -> q_out [tokens][q_heads*128], k_out/v_out
 * [tokens][kv_heads*128]. The per-head sum of squares runs in this build's canonical
 * order (see ora_head_sum_squares). */
void ora_rope_qknorm_f16(int64_t tokens, int64_t row_stride, int64_t q_heads, int64_t kv_heads,
                         int64_t k_offset, float eps, const uint16_t *qkv, const float *q_scale,
                         const float *k_scale, const float *cos_t, const float *sin_t,
                         uint16_t *q_out, uint16_t *k_out, uint16_t *v_out);
float ora_head_sum_squares(const uint16_t *h_head);

/* kernels/native/v_transpose.loom: x [rows][width] -> out [width][capacity]; columns
 * at or past rows untouched. */
void ora_v_transpose(int64_t rows, int64_t width, int64_t capacity, const uint16_t *x,
                     uint16_t *out);

/* kernels/attention_gqa_lds_f16_wmma.loom: grouped-query attention, query head h on
 * kv head h/group (group 4 in the reference kernel), online softmax over key tiles of `key_tile` keys (16 in the reference
 * kernel), weights rounded to f16 for the PV product. vt is V^T [kv_stride][capacity].
 * Writes out rows < rows_out. */
void ora_attention_f16(int64_t tokens, int64_t rows_out, int64_t capacity, int64_t q_stride,
                       int64_t kv_stride, int64_t out_stride, int64_t kv_heads, int64_t group,
                       float scale, int64_t key_tile, const uint16_t *q, const uint16_t *k,
                       const uint16_t *vt, uint16_t *out, int threads);

int ora_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
