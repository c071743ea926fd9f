/*
 * krea2_w8a8.h -- the C ABI of the MI355X (gfx950) W8A8 transformer-product path.
 *
 * One entry point per reference kernel, with the reference's positional buffer
 * bindings in the reference's order, its compile-time configuration passed as a
 * struct (one field per `config.decl`), and its one runtime scalar (`tokens` or
 * `m_size`). Every pointer is device memory the caller owns. GEMMs whose output
 * tiles would leave most CUs idle split K and keep int32 partial sums in a split-K
 * workspace: the caller's, registered per stream with k2w8_gemm_set_workspace, or else
 * one the library allocates per (device, stream) on the first such call outside a
 * stream capture (k2w8_gemm_workspace_bytes() bytes, kept until the process ends; under
 * capture, without either, the call runs unsplit). A recorded block graph owns its own
 * workspace. `stream` is a hipStream_t (NULL: the null stream). Calls enqueue work and
 * return; they do not synchronise.
 *
 * Data types on the buffers:
 *   f16 / bf16 activations: 16-bit IEEE half / bfloat16 bit patterns
 *   int8 operands: row-major [rows][stride] bytes, K contiguous
 *   scales, norm/modulation vectors, residual gates: float32
 *
 * Return codes preserve the reference's three-way error split
 * (src/error.rs:11-29): caller-correctable arguments, host-side contract
 * violations, and runtime (HIP) failures. k2w8_last_error() names the problem.
 */
#ifndef KREA2_W8A8_H
#define KREA2_W8A8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define K2W8_OK 0
#define K2W8_INVALID_ARGUMENT (-1) /* Error::InvalidArgument */
#define K2W8_INTERNAL (-2)         /* Error::Internal */
#define K2W8_RUNTIME (-3)          /* Error::Runtime (a hipError_t) */

/* The ABI revision this header describes. */
#define K2W8_ABI_VERSION 3
int k2w8_abi_version(void);

/* Message of the last failure on the calling thread ("" after success). */
const char *k2w8_last_error(void);

/* kernels/prepare_norm_i8.loom:11-16 (width, out_stride, eps). */
typedef struct k2w8_prepare_norm_cfg {
  int64_t width;      /* K; multiple of 256, 256..32768 */
  int64_t out_stride; /* q row pitch in bytes; multiple of 64, >= width */
  float eps;
} k2w8_prepare_norm_cfg;

/* kernels/prepare_plain_i8.loom:10-13 (width, out_stride). */
typedef struct k2w8_prepare_plain_cfg {
  int64_t width;
  int64_t out_stride;
} k2w8_prepare_plain_cfg;

/* kernels/prepare_gated_i8.loom:11-16 (width, out_stride, gate_stride). */
typedef struct k2w8_prepare_gated_cfg {
  int64_t width;
  int64_t out_stride;
  int64_t gate_stride; /* gate row pitch in elements; multiple of 8, >= width */
} k2w8_prepare_gated_cfg;

/* kernels/gemm_i8_256.loom:14-22 (k_size, n_size, k_stride, m_group), plus
 * kernels/gemm_i8_resid_256x256.loom:26-27 (schedule_rows). m_group and
 * schedule_rows are scheduling hints: they never change results. */
typedef struct k2w8_gemm_cfg {
  int64_t k_size;   /* K; multiple of 128, 128..65536 */
  int64_t n_size;   /* N; multiple of 128, 128..32768 (SwiGLU: 2 x outputs) */
  int64_t k_stride; /* operand row pitch in bytes; multiple of 64, >= k_size */
  int64_t m_group;  /* m-tiles per raster group, 1..4 */
  int64_t schedule_rows;
} k2w8_gemm_cfg;

/*
 * prepare_norm: replaces krea2_prepare_norm_i8 (kernels/prepare_norm_i8.loom:18-22),
 * bound by Session::block (src/session/mod.rs:682-700).
 *   h          bf16 [tokens][width]
 *   norm_scale f32 [width]  (applied as 1 + norm_scale)
 *   mod_scale  f32 [width]  (applied as 1 + mod_scale)
 *   mod_shift  f32 [width]
 *   q          int8 [tokens][out_stride] (bytes >= width untouched)
 *   q_scale    f32 [tokens]
 */
int k2w8_prepare_norm_i8(void *stream, const k2w8_prepare_norm_cfg *cfg, int64_t tokens,
                         const void *h, const float *norm_scale, const float *mod_scale,
                         const float *mod_shift, int8_t *q, float *q_scale);

/*
 * prepare_plain: replaces krea2_prepare_plain_i8 (kernels/prepare_plain_i8.loom:15-19),
 * bound by Session::block (src/session/mod.rs:815-826) and Quantized::forward
 * (src/training/quantized.rs:71-80).
 *   h f16 [tokens][width] -> q int8 [tokens][out_stride], q_scale f32 [tokens]
 */
int k2w8_prepare_plain_i8(void *stream, const k2w8_prepare_plain_cfg *cfg, int64_t tokens,
                          const void *h, int8_t *q, float *q_scale);

/*
 * prepare_gated: replaces krea2_prepare_gated_i8 (kernels/prepare_gated_i8.loom:18-22),
 * bound by Session::block (src/session/mod.rs:757-770).
 *   attn f16 [tokens][width], gate f16 [tokens][gate_stride]
 *   -> q int8 [tokens][out_stride], q_scale f32 [tokens]
 * The first call on a device builds the device's 128 KiB table of bf16(sigmoid(g))
 * over all f16 gates (a static device array) on `stream` and synchronises `stream`
 * once; that first call must not be inside a stream capture (k2w8_blocks_record sets
 * the device up before it captures).
 */
int k2w8_prepare_gated_i8(void *stream, const k2w8_prepare_gated_cfg *cfg, int64_t tokens,
                          const void *attn, const void *gate, int8_t *q, float *q_scale);

/*
 * gemm_i8: replaces krea2_gemm_i8_256 (kernels/gemm_i8_256.loom:24-36), bound by
 * Session::gemm (src/session/mod.rs:650-669) and Quantized::forward
 * (src/training/quantized.rs:81-101).
 *   a       int8 [m][k_stride], w int8 [n_size][k_stride]
 *   scale   f32 [n_size] (per output channel), a_scale f32 [m] (per token)
 *   c       f16 [m][n_size] = f16(bf16((f32(acc) * scale[n]) * a_scale[m]))
 */
int k2w8_gemm_i8(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                 const int8_t *w, const float *scale, const float *a_scale, void *c);

/*
 * gemm_i8_resid: replaces krea2_gemm_i8_resid_256 (kernels/gemm_i8_resid_256.loom:24-36).
 *   c    bf16 [m][n_size], read and written in place:
 *        c = bf16(c + bf16(gate[n] * bf16((f32(acc) * scale[n]) * a_scale[m])))
 *   gate f32 [n_size]
 */
int k2w8_gemm_i8_resid(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                       const int8_t *w, const float *scale, const float *a_scale, void *c,
                       const float *gate);

/* Replaces krea2_gemm_i8_resid_256x256 (kernels/gemm_i8_resid_256x256.loom), the
 * down projection's kernel (src/kernels/shape.rs:68-90). Same bindings and
 * results as k2w8_gemm_i8_resid. */
int k2w8_gemm_i8_resid_256x256(void *stream, const k2w8_gemm_cfg *cfg, int64_t m,
                               const int8_t *a, const int8_t *w, const float *scale,
                               const float *a_scale, void *c, const float *gate);

/*
 * gemm_i8_swiglu: replaces krea2_gemm_i8_swiglu_256 (kernels/gemm_i8_swiglu_256.loom:24-36).
 *   w rows interleaved in 16-row groups [gate o..o+15 | up o..o+15]
 *   (src/checkpoint/plan.rs:193-208), scale likewise.
 *   c f16 [m][n_size/2]: c[m][o] = f16(bf16(bf16(g*sigmoid(g)) * u)),
 *   g = bf16((f32(acc[gc]) * scale[gc]) * a_scale[m]), gc = (o/16)*32 + o%16,
 *   u likewise at gc + 16.
 */
int k2w8_gemm_i8_swiglu(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                        const int8_t *w, const float *scale, const float *a_scale, void *c);

/*
 * gemm_i8_bias: no reference counterpart (the reference's W8A8 GEMMs carry no
 * bias); the plain GEMM with an f16 bias added before the bf16 boundary:
 *   c = f16(bf16((f32(acc) * scale[n]) * a_scale[m] + bias[n]))
 */
int k2w8_gemm_i8_bias(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                      const int8_t *w, const float *scale, const float *a_scale,
                      const void *bias, void *c);

/*
 * gemm_i8_acc: no reference counterpart; the exact int32 accumulators
 * acc[m][n] = sum_{k < k_size} a[m][k] * w[n][k] with no epilogue. These are the
 * partial sums a K-sharded (row-parallel) projection exchanges before its
 * epilogue: integer addition is associative, so the exchange stays bit-exact.
 *   acc int32 [m][n_size]
 */
int k2w8_gemm_i8_acc(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                     const int8_t *w, int32_t *acc);

/*
 * Split-K workspace of a stream. Replaces the session-owned GEMM workspaces of
 * src/session/mod.rs:321-340 (the reference's session allocates every buffer up front
 * and its launches allocate nothing).
 *
 * gemm_set_workspace: GEMM calls on `stream` (current device) keep their split-K
 * partial sums in `workspace` (`bytes` of device memory, 256-byte aligned, >= 256)
 * instead of a library allocation, so they never allocate, also under stream capture
 * (a captured split-K GEMM then splits as an eager one does). The number of K slices is
 * capped by what fits: a smaller workspace means fewer slices, never a failure. The
 * caller keeps the memory alive while it is registered and while work already enqueued
 * may use it; calls on one stream are ordered, so they may share it. A null workspace
 * removes the registration (the library's own buffer is used again).
 * gemm_workspace_bytes: the size of the library's own per-stream workspace, which
 * holds every split this build chooses.
 */
int k2w8_gemm_set_workspace(void *stream, void *workspace, int64_t bytes);
int64_t k2w8_gemm_workspace_bytes(void);

/*
 * gemm_i8_noalloc: no counterpart in the reference. For callers that cannot allocate
 * (code under graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * k2w8_gemm_i8 with the same arguments and bit-identical results, whose split-K
 * partial sums go to a 16 MiB static device array of the library (one per device,
 * held until the process ends) instead of any workspace, so no call allocates
 * device memory. A shape that would split K into slices of which two do not fit
 * (2 * m * n_size * 4 bytes > 16 MiB) is refused with INVALID_ARGUMENT; on a 256-CU
 * MI355X the split rule never picks one (it splits only when the 128x128 tiles cover
 * at most half the CUs, so m * n_size <= 2^21). Every call on a device shares that device's
 * array. Eager calls that split K are ordered on the device: each one's stream waits
 * (hipStreamWaitEvent, no host wait) for the previous such call's work, whatever its
 * stream. Calls recorded into a graph are ordered by the graph; replays of two graphs
 * that both hold such a call must not overlap (on different streams), or they race on
 * the array. The first call on a device looks up the array's address there and creates
 * the ordering event; no call allocates device memory.
 */
int k2w8_gemm_i8_noalloc(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                         const int8_t *w, const float *scale, const float *a_scale, void *c);

/*
 * gemm_choose: no counterpart in the reference. Which kernel the GEMM entry points run
 * for a shape on a device with `cus` compute units and a split-K workspace of
 * `workspace_bytes` (the library's own: k2w8_gemm_workspace_bytes()), without launching
 * anything: the rule launch_gemm applies, for tuning reports and host-side tests.
 * `epilogue` is 0 plain, 1 residual, 2 SwiGLU, 3 bias, 4 int32 accumulators.
 * `workspace_required` nonzero describes a call whose workspace is fixed at
 * `workspace_bytes` and may not be replaced (gemm_i8_noalloc: its static scratch); a shape
 * such a call refuses reports kernel -1. The library's per-stream workspace is not
 * available inside a stream capture unless one was registered (gemm_set_workspace) or
 * a recording installed it: pass workspace_bytes = 0 to see what a captured call runs.
 */
typedef struct k2w8_gemm_choice {
  int32_t kernel;  /* 0 few-token kernel, 1 tile kernel, 2 256x256 tiles then the last
                      columns as 128x128 tiles, 3 split K over 128x128 tiles + reduction,
                      -1 refused (workspace_required, two slices do not fit) */
  int32_t tile_m, tile_n; /* kernels 1-3: the workgroup tile (kernel 2: 256x256) */
  int32_t stages;         /* kernels 1-3: LDS stages of the tile kernel */
  int64_t n_big;          /* kernel 2: the columns that run as 256x256 tiles */
  int32_t split_steps;    /* kernel 3: 128-byte K steps per slice */
  int32_t splits;         /* kernel 3: slices */
} k2w8_gemm_choice;
int k2w8_gemm_choose(int32_t epilogue, int64_t m, const k2w8_gemm_cfg *cfg, int64_t cus,
                     int64_t workspace_bytes, int32_t workspace_required, k2w8_gemm_choice *out);

/*
 * linear_norm_i8 / linear_plain_i8: one call for a projection:
 * prepare_norm_i8 (resp. prepare_plain_i8) of h into q / q_scale, then
 * gemm_i8 of q with w into c, as one call. Replaces the prepare -> gemm_i8 launch pair
 * of Session::block and Quantized::forward (src/session/mod.rs:671-711,
 * src/training/quantized.rs:66-105). The arguments are the two entry points' own (the
 * GEMM's k_size / k_stride must equal the prepare's width / out_stride, its m is
 * `tokens`), and the outputs are bit-identical to calling them in turn; q and q_scale
 * are written as well. They run as the two launches. With the environment variable
 * K2W8_LINEAR_ONE_LAUNCH=1, the wide-tile shapes (whole rounds of 256x192 tiles, width
 * <= 3072) run instead in one persistent launch with a grid-wide barrier between the
 * phases (one workgroup per CU); it gives the same bits but measured slower, so it is
 * not the default. The barrier's count is the launch's own: the first 256 bytes of the
 * stream's split-K workspace, cleared by a small kernel launched before it (a capture
 * with no workspace installed or registered records the two launches instead). Its
 * wait is bounded (K2W8_FUSED_BARRIER_POLLS polls, default 16384); a workgroup that
 * gives up (other work holding CUs, e.g. a one-launch call on another stream) prepares
 * the rows of its own tiles again before each tile, so the output stays exact.
 */
int k2w8_linear_norm_i8(void *stream, const k2w8_prepare_norm_cfg *cfg, const k2w8_gemm_cfg *gemm,
                        int64_t tokens, const void *h, const float *norm_scale,
                        const float *mod_scale, const float *mod_shift, int8_t *q,
                        float *q_scale, const int8_t *w, const float *scale, void *c);
int k2w8_linear_plain_i8(void *stream, const k2w8_prepare_plain_cfg *cfg, const k2w8_gemm_cfg *gemm,
                         int64_t tokens, const void *h, int8_t *q, float *q_scale,
                         const int8_t *w, const float *scale, void *c);

/*
 * The block's other prepare -> GEMM pairs as one call each (always two launches),
 * with the arguments of the two entry points they chain and the same bits:
 *   linear_gated_resid_i8: prepare_gated_i8 -> gemm_i8_resid (the attention output
 *     projection, src/session/mod.rs:757-783);
 *   linear_norm_swiglu_i8: prepare_norm_i8 -> gemm_i8_swiglu (gate|up,
 *     src/session/mod.rs:785-813);
 *   linear_plain_resid_i8: prepare_plain_i8 -> gemm_i8_resid (down,
 *     src/session/mod.rs:815-840).
 * `gate_in` is the gated prepare's gate, `gate` the residual's per-channel gate, `x`
 * the bf16 residual updated in place.
 */
int k2w8_linear_gated_resid_i8(void *stream, const k2w8_prepare_gated_cfg *cfg, const k2w8_gemm_cfg *gemm,
                               int64_t tokens, const void *attn, const void *gate_in, int8_t *q,
                               float *q_scale, const int8_t *w, const float *scale, void *x,
                               const float *gate);
int k2w8_linear_norm_swiglu_i8(void *stream, const k2w8_prepare_norm_cfg *cfg, const k2w8_gemm_cfg *gemm,
                               int64_t tokens, const void *h, const float *norm_scale,
                               const float *mod_scale, const float *mod_shift, int8_t *q,
                               float *q_scale, const int8_t *w, const float *scale, void *c);
int k2w8_linear_plain_resid_i8(void *stream, const k2w8_prepare_plain_cfg *cfg, const k2w8_gemm_cfg *gemm,
                               int64_t tokens, const void *h, int8_t *q, float *q_scale,
                               const int8_t *w, const float *scale, void *x, const float *gate);

/*
 * lora_transport: replaces krea2_lora_transport (kernels/native/lora_transport.loom:5-41),
 * the 16-bit format change around the W8A8 projection of src/training/quantized.rs:66-105.
 * Each element is widened exactly to f32 and rounded (nearest even) to the other format.
 *   direction 1 (the reference's `reverse` = 1): x bf16 [count] -> out f16 [count]
 *   direction 2 (`reverse` = 2):                 x f16 [count]  -> out bf16 [count]
 * count in 1..2^30-1 (:13); x and out 16-byte aligned.
 */
int k2w8_lora_transport(void *stream, int direction, int64_t count, const void *x, void *out);

/*
 * sigmoid_f32: none in the reference (a check of this build's numerics). Evaluates,
 * elementwise, the device sigmoid 1 / (1 + exp(-x)) that prepare_gated_i8 and the
 * SwiGLU epilogue use, so its bits can be compared with the CPU definition.
 *   x f32 [count] -> out f32 [count]; count in 1..2^32-1.
 */
int k2w8_sigmoid_f32(void *stream, int64_t count, const float *x, float *out);

/* Shape of a ConvRot projection (src/training/quantized.rs:8-14). */
typedef struct k2w8_quantized_cfg {
  int64_t inputs;  /* K: a multiple of 256 (prepare width rules) */
  int64_t outputs; /* N: a multiple of 128 */
  int64_t pitch;   /* row pitch of weight and quantized rows (k2w8_shape_gemm_pitch(inputs)) */
} k2w8_quantized_cfg;

/*
 * quantized_forward: Quantized::forward (src/training/quantized.rs:51-112), the
 * secondary caller of the path, as one call issuing its four launches in order on
 * `stream`: transport bf16 -> f16, prepare_plain_i8, gemm_i8, transport f16 -> bf16.
 * The caller owns every buffer, including the workspaces the reference takes from its
 * pool (:55-58):
 *   x bf16 [rows][inputs], weight int8 [outputs][pitch], scales f32 [outputs],
 *   transport f16 [rows * inputs], quantized int8 [rows][pitch], q_scales f32 [rows],
 *   out_f16 f16 [rows][outputs], out bf16 [rows][outputs].
 */
int k2w8_quantized_forward(void *stream, const k2w8_quantized_cfg *cfg, int64_t rows,
                           const void *x, const int8_t *weight, const float *scales,
                           void *transport, int8_t *quantized, float *q_scales, void *out_f16,
                           void *out);

/* ---- The attention step of a block (src/session/mod.rs:714-755) ---- */

/* kernels/rope_qknorm_f16.loom:12-20 */
typedef struct k2w8_rope_qknorm_cfg {
  int64_t row_stride; /* qkv row pitch in elements; multiple of 128, 128..65536 */
  int64_t q_heads;    /* 1..256 */
  int64_t kv_heads;   /* 1..256 */
  int64_t k_offset;   /* first k column; multiple of 128, 128..65536 */
  float eps;
} k2w8_rope_qknorm_cfg;

/*
 * rope_qknorm_f16: replaces krea2_rope_qknorm_f16 (kernels/rope_qknorm_f16.loom:22-159).
 * Bindings in the reference's order (:24):
 *   qkv f16 [tokens][row_stride]: q heads at column 0, k heads at k_offset, v heads at
 *       k_offset + kv_heads*128 (the fused qkvg GEMM output)
 *   q_scale, k_scale f32 [128]: zero-centred RMSNorm scales (multiplier 1 + scale)
 *   cos, sin f32 [tokens][128]
 *   q_out f16 [tokens][q_heads*128], k_out, v_out f16 [tokens][kv_heads*128]
 * Per head: x = bf16(h / sqrt(mean(h^2) + eps) * (1 + scale[c])), then the rotary
 * pairs (2i, 2i+1) -> bf16(x0 cos - x1 sin), bf16(x1 cos + x0 sin), stored as f16;
 * v heads are copied. tokens in 1..2^20; every buffer 16-byte aligned.
 */
int k2w8_rope_qknorm_f16(void *stream, const k2w8_rope_qknorm_cfg *cfg, int64_t tokens,
                         const void *qkv, const float *q_scale, const float *k_scale,
                         const float *cos, const float *sin, void *q_out, void *k_out,
                         void *v_out);

/* kernels/native/v_transpose.loom:7-9 */
typedef struct k2w8_v_transpose_cfg {
  int64_t width;        /* multiple of 32, 32..65536 */
  int64_t row_capacity; /* multiple of 32, 32..2^20 */
} k2w8_v_transpose_cfg;

/*
 * v_transpose: replaces krea2_v_transpose (kernels/native/v_transpose.loom:11-90,
 * src/session/v_transpose.rs): x f16 [rows][width] -> out f16 [width][row_capacity].
 * Columns at or past `rows` are not written: the caller keeps them zero (the attention
 * kernel reads them). rows in 1..row_capacity; x and out 16-byte aligned.
 */
int k2w8_v_transpose(void *stream, const k2w8_v_transpose_cfg *cfg, int64_t rows, const void *x,
                     void *out);

/* kernels/attention_gqa_lds_f16_wmma.loom:18-28 */
typedef struct k2w8_attention_cfg {
  int64_t q_stride;       /* q row pitch in elements; multiple of 128, 128..32768 */
  int64_t kv_stride;      /* k row pitch and V^T rows; multiple of 128, 128..32768 */
  int64_t out_stride;     /* out row pitch; multiple of 128, 128..32768 */
  int64_t tokens;         /* keys and queries: 16..65536 */
  int64_t token_capacity; /* rows of q and k, columns of V^T: multiple of 16, >= tokens + 16 */
  float scale;            /* score scale, 1/sqrt(128) in production */
} k2w8_attention_cfg;

/*
 * attention_f16: replaces krea2_attention_gqa_lds_f16_wmma and its 32-query twin
 * (kernels/attention_gqa_lds_f16_wmma.loom:30-380, _q32.loom), non-causal grouped-query
 * attention with four query heads per key-value head (query head h reads kv head h/4).
 * Bindings in the reference's order (:35):
 *   q f16 [token_capacity][q_stride], k f16 [token_capacity][kv_stride],
 *   v = V^T f16 [kv_stride][token_capacity] (as k2w8_v_transpose writes it),
 *   out f16 [token_count][out_stride]
 * out[t][h*128 + c] = sum_j softmax_j(scale * q_t.k_j) v_j[c] over keys j < tokens, with
 * fp16 products, f32 accumulation and an f32 online softmax whose weights are rounded
 * to f16 for the PV product. Rows t < min(tokens, token_count) are written. Rows of q
 * and k and columns of V^T past `tokens` must be zero. kv_head_count in 1..
 * kv_stride/128, with 4 * kv_head_count * 128 <= q_stride and <= out_stride.
 */
int k2w8_attention_f16(void *stream, const k2w8_attention_cfg *cfg, int64_t token_count,
                       int64_t kv_head_count, const void *q, const void *k, const void *v,
                       void *out);

/*
 * attention_f16_grouped: k2w8_attention_f16 with `group` query heads per key-value head
 * (1, 2 or 4; query head h reads kv head h / group). An extension: the reference kernel
 * fixes the group at 4; the block entry points use this for head layouts whose ratio
 * differs. Same bindings and rules, with group * kv_head_count * 128 in place of
 * 4 * kv_head_count * 128.
 */
int k2w8_attention_f16_grouped(void *stream, const k2w8_attention_cfg *cfg, int64_t token_count,
                               int64_t kv_head_count, int64_t group, const void *q, const void *k,
                               const void *v, void *out);

/* ---- Checkpoint upload (host code; src/checkpoint/, src/session/weights.rs) ---- */

/* Tensor element types of a .safetensors header. */
enum {
  K2W8_DTYPE_OTHER = 0,
  K2W8_DTYPE_I8 = 1,
  K2W8_DTYPE_F32 = 2,
  K2W8_DTYPE_BF16 = 3,
  K2W8_DTYPE_F16 = 4,
  K2W8_DTYPE_U8 = 5,
  K2W8_DTYPE_I32 = 6
};

/* A memory-mapped .safetensors file, indexed under its tensors' names with a
 * whole-model save's shared prefix removed (src/checkpoint/file.rs:64-130). */
typedef struct k2w8_checkpoint k2w8_checkpoint;

/* One tensor of a checkpoint (file.rs:12-21): its bytes point into the mapping and
 * live as long as the checkpoint. */
typedef struct k2w8_tensor {
  int32_t dtype; /* K2W8_DTYPE_* */
  int32_t ndim;
  int64_t shape[8];
  const void *data;
  int64_t nbytes;
} k2w8_tensor;

/* Checkpoint::open (file.rs:86-106): a name not ending in .safetensors, a header longer
 * than the file, or a tensor reaching past the data is INVALID_ARGUMENT. */
int k2w8_checkpoint_open(const char *path, k2w8_checkpoint **out);
void k2w8_checkpoint_close(k2w8_checkpoint *file);
/* Checkpoint::block_count (file.rs:124-129). */
int64_t k2w8_checkpoint_block_count(const k2w8_checkpoint *file);
/* Checkpoint::get (file.rs:114-120); a missing name is INVALID_ARGUMENT. */
int k2w8_checkpoint_tensor(const k2w8_checkpoint *file, const char *name, k2w8_tensor *out);

/* The device layout of a checkpoint's ConvRot block weights (src/checkpoint/plan.rs). */
typedef struct k2w8_plan k2w8_plan;

/* One destination of the plan (plan.rs:24-41). */
typedef struct k2w8_span {
  int64_t device_offset;    /* in the single weights allocation, 256-byte aligned */
  int64_t device_bytes;     /* bytes it occupies at the device pitch */
  int64_t rows;             /* rows copied from the file (0: bytes assembled on the host) */
  int64_t row_bytes;        /* bytes per row in the file */
  int64_t device_row_bytes; /* bytes per row on the device (the GEMM pitch) */
  int64_t file_bytes;       /* Span::file_bytes (plan.rs:43-48) */
  int64_t segments;         /* checkpoint row ranges that fill it */
} k2w8_span;

/* Plan::for_checkpoint (plan.rs:88-143): per block, qkvg.{q,s} = wq|wk|wv|attn.gate rows
 * and scales, wo.{q,s}, down.{q,s}, gu.{q,s} = mlp.gate and mlp.up interleaved 16 rows at
 * a time, and the f32 vectors prenorm, postnorm, qnorm, knorm (bf16 upcast exactly). */
int k2w8_plan_for_checkpoint(const k2w8_checkpoint *file, k2w8_plan **out);
void k2w8_plan_free(k2w8_plan *plan);
int64_t k2w8_plan_total_bytes(const k2w8_plan *plan);
int64_t k2w8_plan_layers(const k2w8_plan *plan);
/* The spans in name order (the order their offsets were assigned in). */
int64_t k2w8_plan_span_count(const k2w8_plan *plan);
const char *k2w8_plan_span_name(const k2w8_plan *plan, int64_t index);
/* Plan::span (plan.rs:146-149); an unknown name is INVALID_ARGUMENT. */
int k2w8_plan_span(const k2w8_plan *plan, const char *name, k2w8_span *out);

/* Weights::upload (src/session/weights.rs:48-100): zero `device` (at least
 * k2w8_plan_total_bytes bytes), then place every span's rows at its device pitch from
 * the mapped file, on `stream`; returns after the stream has drained. */
int k2w8_plan_upload(void *stream, const k2w8_plan *plan, const k2w8_checkpoint *file,
                     void *device, int64_t device_bytes);

/* ---- The W8A8 stages of a transformer block (src/session/mod.rs) ---- */

/* Specialisation of a block (src/kernels/blocks.rs:38-107; production: hidden 6144,
 * inter 16384, qkvg 15360, gate_offset 9216, eps 1e-5). */
typedef struct k2w8_block_cfg {
  int64_t tokens;      /* rows of x and of every activation buffer in use */
  int64_t hidden;      /* residual width, K of qkvg/gu/wo and N of wo/down */
  int64_t inter;       /* MLP width, K of down (gu has 2 * inter interleaved rows) */
  int64_t qkvg;        /* columns of the fused q|k|v|gate output */
  int64_t gate_offset; /* first column of the gate half (src/session/mod.rs:45) */
  float eps;           /* RMSNorm epsilon */
} k2w8_block_cfg;

/* One block's resident operands (the plan's blocks.<i>.* spans). */
typedef struct k2w8_block_weights {
  const int8_t *qkvg_q; const float *qkvg_s;
  const int8_t *wo_q;   const float *wo_s;
  const int8_t *gu_q;   const float *gu_s;
  const int8_t *down_q; const float *down_s;
  const float *prenorm; const float *postnorm;
  const float *qnorm;   const float *knorm;  /* f32 [128]: rope_qknorm's q_scale, k_scale */
} k2w8_block_weights;

/* The session's workspaces (src/session/mod.rs:321-340), owned by the caller. */
typedef struct k2w8_block_buffers {
  void *x;           /* bf16 [tokens][hidden], the residual stream, in place */
  int8_t *a_q;       /* int8 [tokens][pitch(max(hidden, inter))] */
  float *a_s;        /* f32 [tokens] */
  void *fused;       /* f16 [tokens][qkvg] */
  void *attn_gu;     /* f16 [tokens][max(hidden, inter)]: attention output, then SwiGLU output */
  const float *mods; /* f32 [layers][6][hidden]: prescale, preshift, pregate, postscale,
                        postshift, postgate (src/session/mod.rs:133-138) */
  /* The attention step's workspaces (src/session/mod.rs:327-341), capacity =
   * k2w8_shape_capacity(tokens), kv = (gate_offset - hidden) / 2 columns of k and of v.
   * With q NULL the block runs its W8A8 stages only and the caller leaves the attention
   * output in attn_gu between k2w8_block_pre_attention and k2w8_block_post_attention. */
  void *q;          /* f16 [capacity][hidden], rows past tokens zero */
  void *k;          /* f16 [capacity][kv], rows past tokens zero */
  void *v;          /* f16 [capacity][kv] */
  void *vt;         /* f16 [kv][capacity], columns past tokens zero */
  const float *cos; /* f32 [tokens][128] */
  const float *sin; /* f32 [tokens][128] */
} k2w8_block_buffers;

/* Session::block (src/session/mod.rs:671-711), up to the attention: prepare_norm_i8
 * with the block's prenorm and modulation rows 0/1, then gemm_qkvg into `fused`. */
int k2w8_block_pre_attention(void *stream, const k2w8_block_cfg *cfg, int64_t index,
                             const k2w8_block_weights *weights, const k2w8_block_buffers *buffers);
/* Session::block (:713-755), the attention step: rope_qknorm_f16 over the q and k heads
 * of `fused` (weights qnorm/knorm, cos/sin) into q/k/v, the V transpose into vt, and
 * f16 attention into attn_gu [tokens][hidden] with scale 1/sqrt(128). Query heads
 * hidden/128, key-value heads kv/128, in a ratio of 1, 2 or 4; tokens >= 16. */
int k2w8_block_attention(void *stream, const k2w8_block_cfg *cfg, int64_t index,
                         const k2w8_block_weights *weights, const k2w8_block_buffers *buffers);
/* Session::block (:756-839), after the attention (whose output the caller left in
 * attn_gu): prepare_gated_i8 over the gate half, gemm_wo + residual (gate = row 2),
 * prepare_norm_i8 (postnorm, rows 3/4), gemm_gu + SwiGLU into attn_gu,
 * prepare_plain_i8, gemm_down + residual (gate = row 5). */
int k2w8_block_post_attention(void *stream, const k2w8_block_cfg *cfg, int64_t index,
                              const k2w8_block_weights *weights, const k2w8_block_buffers *buffers);

/* A recorded block loop (src/session/mod.rs:596-616): `layers` blocks, weights[i] for
 * block i, captured once from `stream` (a created stream) into a hipGraph over the
 * same buffers, replayed by k2w8_graph_launch. Each block is pre_attention, the
 * attention step when buffers->q is set, then post_attention. */
typedef struct k2w8_graph k2w8_graph;
int k2w8_blocks_record(void *stream, const k2w8_block_cfg *cfg, int64_t layers,
                       const k2w8_block_weights *weights, const k2w8_block_buffers *buffers,
                       k2w8_graph **out);
int k2w8_graph_launch(void *stream, k2w8_graph *graph);
void k2w8_graph_free(k2w8_graph *graph);

/* The stage profile (src/session/mod.rs:449-479, 618-647): one eager pass over `layers`
 * blocks with events around every launch; stage_us[k] accumulates the microseconds of
 * stage k (labels from k2w8_block_stage_label) over all blocks, -1 for the attention
 * stages when buffers->q is NULL. */
int k2w8_blocks_profile(void *stream, const k2w8_block_cfg *cfg, int64_t layers,
                        const k2w8_block_weights *weights, const k2w8_block_buffers *buffers,
                        double *stage_us, int64_t stage_count);
int64_t k2w8_block_stage_count(void);
const char *k2w8_block_stage_label(int64_t index);

/*
 * probe_mfma_i8: a measurement aid with no counterpart in the reference. Back-to-back
 * v_mfma_i32_32x32x32_i8 on operands held in registers (pseudo-random bytes from
 * `seed` when `random` is non-zero, else bytes of 1), `blocks` workgroups of four waves,
 * `iters` steps of eight MFMAs per wave: 2^21 * blocks * iters ops. The INT8 MFMA rate
 * the chip holds under its power limit, which the tile GEMM is measured against.
 * out: int32 [blocks * 256], each lane's accumulator sum (with bytes of 1:
 * 4096 * iters).
 */
int k2w8_probe_mfma_i8(void *stream, int64_t blocks, int64_t iters, int32_t random, uint32_t seed,
                       int32_t *out);

/*
 * Configuration checks alone, as the reference's config.decl ranges constrain each
 * kernel (kernels/gemm_i8_256.loom:14-22, kernels/prepare_norm_i8.loom:11-16,
 * kernels/prepare_plain_i8.loom:10-13, kernels/prepare_gated_i8.loom:11-16): K2W8_OK,
 * or K2W8_INVALID_ARGUMENT with the reason in k2w8_last_error(). The entry points run
 * the same checks. Every configuration the reference accepts passes, except GEMM
 * k_size values that are odd multiples of 64 (this build's K step is 128 bytes; no
 * production shape has one) and a gated gate_stride below the width.
 */
int k2w8_validate_gemm_cfg(const k2w8_gemm_cfg *cfg);
int k2w8_validate_prepare_norm_cfg(const k2w8_prepare_norm_cfg *cfg);
int k2w8_validate_prepare_plain_cfg(const k2w8_prepare_plain_cfg *cfg);
int k2w8_validate_prepare_gated_cfg(const k2w8_prepare_gated_cfg *cfg);

/* Launch-shape rules of src/kernels/shape.rs:7-112. */
/* The size arguments are the reference's usize values: for 0..2^40 the rules below
 * answer as the reference does; outside that domain they return -1. */
int64_t k2w8_shape_gemm_pitch(int64_t k);    /* shape.rs:105-107 */
int64_t k2w8_shape_capacity(int64_t tokens); /* shape.rs:12-16 */
int64_t k2w8_shape_gemm_grid_rows(int64_t tokens); /* shape.rs:110-112 */
int k2w8_shape_gemm_schedule_rows(int64_t tokens); /* shape.rs:97-99 */
int64_t k2w8_shape_gemm_rows(void);    /* GEMM_ROWS, shape.rs:36 */
int64_t k2w8_shape_gemm_m_group(void); /* GEMM_M_GROUP, shape.rs:93 */
int64_t k2w8_shape_tokens_min(void);   /* TOKENS, shape.rs:8 */
int64_t k2w8_shape_tokens_max(void);

#ifdef __cplusplus
}
#endif
#endif
