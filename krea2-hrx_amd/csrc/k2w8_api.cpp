// The C ABI (include/krea2_w8a8.h): argument validation mirroring the reference's
// `config.decl` constraints, the launch-shape rules of src/kernels/shape.rs, and
// the three-way error split of src/error.rs:11-29.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "krea2_w8a8.h"
#include "k2w8_internal.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return K2W8_OK;
}

int runtime(const char *stage, hipError_t e) {
  return fail(K2W8_RUNTIME, "%s: %s", stage, hipGetErrorString(e));
}

// Large dynamic LDS must be enabled per kernel once per process (and device).
int ensure_configured(const char *stage) {
  static std::once_flag once;
  static hipError_t status = hipSuccess;
  static const char *what = "";
  std::call_once(once, [] {
    what = "enabling the prepare kernels' LDS";
    status = k2w8::configure_prepare_lds();
    if (status == hipSuccess) {
      what = "enabling the GEMM kernels' LDS";
      status = k2w8::configure_gemm_lds();
    }
  });
  if (status != hipSuccess)
    return fail(K2W8_RUNTIME, "%s: %s: %s", stage, what, hipGetErrorString(status));
  return K2W8_OK;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Token bound of the prepares and GEMMs (kernels/prepare_norm_i8.loom:56, gemm m range).
constexpr int64_t kMaxTokens = 1 << 20;

int check_prepare(const char *stage, int64_t tokens, int64_t width, int64_t out_stride,
                  const void *h, const int8_t *q, const float *q_scale) {
  if (tokens < 1 || tokens > kMaxTokens)
    return fail(K2W8_INVALID_ARGUMENT, "%s: tokens must be 1..%lld, got %lld", stage,
                (long long)kMaxTokens, (long long)tokens);
  if (width < 256 || width > 32768 || width % 256 != 0)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: width must be a multiple of 256 in 256..32768, got %lld", stage,
                (long long)width);
  if (out_stride < width || out_stride > 65536 || out_stride % 64 != 0)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: out_stride must be a multiple of 64 in width..65536, got %lld", stage,
                (long long)out_stride);
  if (!h || !q || !q_scale) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(h, 16) || !aligned(q, 16) || !aligned(q_scale, 4))
    return fail(K2W8_INVALID_ARGUMENT, "%s: h and q must be 16-byte aligned", stage);
  return K2W8_OK;
}

int check_gemm(const char *stage, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
               const int8_t *w, const float *scale, const float *a_scale, const void *c) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  if (cfg->k_size < 128 || cfg->k_size > 65536 || cfg->k_size % 128 != 0)
    return fail(K2W8_INVALID_ARGUMENT, "%s: k_size must be a multiple of 128 in 128..65536, got %lld",
                stage, (long long)cfg->k_size);
  if (cfg->n_size < 128 || cfg->n_size > 32768 || cfg->n_size % 128 != 0)
    return fail(K2W8_INVALID_ARGUMENT, "%s: n_size must be a multiple of 128 in 128..32768, got %lld",
                stage, (long long)cfg->n_size);
  if (cfg->k_stride < cfg->k_size || cfg->k_stride > 65536 || cfg->k_stride % 64 != 0)
    return fail(K2W8_INVALID_ARGUMENT, "%s: k_stride must be a multiple of 64 in k_size..65536, got %lld",
                stage, (long long)cfg->k_stride);
  if (cfg->m_group < 1 || cfg->m_group > 4)
    return fail(K2W8_INVALID_ARGUMENT, "%s: m_group must be 1..4, got %lld", stage,
                (long long)cfg->m_group);
  if (m < 1 || m > 16777216)
    return fail(K2W8_INVALID_ARGUMENT, "%s: m must be 1..16777216, got %lld", stage, (long long)m);
  // 32-bit element offsets inside the kernels.
  if (m * cfg->k_stride >= (int64_t(1) << 31) || cfg->n_size * cfg->k_stride >= (int64_t(1) << 31) ||
      m * cfg->n_size >= (int64_t(1) << 31))
    return fail(K2W8_INVALID_ARGUMENT, "%s: operands exceed 2^31 elements", stage);
  if (!a || !w || !scale || !a_scale || !c) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(scale, 16) || !aligned(c, 16) ||
      !aligned(a_scale, 4))
    return fail(K2W8_INVALID_ARGUMENT, "%s: a, w, scale and c must be 16-byte aligned", stage);
  return K2W8_OK;
}

int run_gemm(const char *stage, int epi, void *stream, const k2w8_gemm_cfg *cfg, int64_t m,
             const int8_t *a, const int8_t *w, const float *scale, const float *a_scale, void *c,
             const float *gate, const void *bias) {
  int rc = check_gemm(stage, cfg, m, a, w, scale, a_scale, c);
  if (rc != K2W8_OK) return rc;
  if (epi == k2w8::kEpiResid && !gate) return fail(K2W8_INVALID_ARGUMENT, "%s: null gate", stage);
  if (epi == k2w8::kEpiBias && !bias) return fail(K2W8_INVALID_ARGUMENT, "%s: null bias", stage);
  if ((gate && !aligned(gate, 16)) || (bias && !aligned(bias, 16)))
    return fail(K2W8_INVALID_ARGUMENT, "%s: gate and bias must be 16-byte aligned", stage);
  if ((rc = ensure_configured(stage)) != K2W8_OK) return rc;
  k2w8::GemmLaunch l;
  l.a = a;
  l.w = w;
  l.w_scale = scale;
  l.a_scale = a_scale;
  l.c = c;
  l.gate = gate;
  l.bias = bias;
  l.m = m;
  l.n = cfg->n_size;
  l.k = cfg->k_size;
  l.lda = cfg->k_stride;
  l.m_group = (int)cfg->m_group;
  hipError_t e = k2w8::launch_gemm(epi, static_cast<hipStream_t>(stream), l);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

}  // namespace

// The error channel for the library's other host sources (k2w8_checkpoint.cpp).
int k2w8_fail_invalid(const char *message) { return fail(K2W8_INVALID_ARGUMENT, "%s", message); }
int k2w8_fail_runtime(const char *stage, hipError_t e) { return runtime(stage, e); }
int k2w8_succeed() { return ok(); }
// The one-time set-up of the launch paths (kernel attributes, device queries), done
// before a stream capture so that none of it happens inside one.
int k2w8_prime_launches() {
  int rc = ensure_configured("blocks_record");
  if (rc != K2W8_OK) return rc;
  (void)k2w8::device_cus();
  // Allocate the split-K workspace now, outside the capture, so recorded GEMMs may
  // split K as eager ones do.
  (void)k2w8::splitk_workspace(nullptr);
  return K2W8_OK;
}

extern "C" {

int k2w8_abi_version(void) { return K2W8_ABI_VERSION; }

const char *k2w8_last_error(void) { return g_last_error.c_str(); }

int k2w8_prepare_norm_i8(void *stream, const k2w8_prepare_norm_cfg *cfg, int64_t tokens,
                         const void *h, const float *norm_scale, const float *mod_scale,
                         const float *mod_shift, int8_t *q, float *q_scale) {
  const char *stage = "prepare_norm_i8";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  int rc = check_prepare(stage, tokens, cfg->width, cfg->out_stride, h, q, q_scale);
  if (rc != K2W8_OK) return rc;
  if (!norm_scale || !mod_scale || !mod_shift)
    return fail(K2W8_INVALID_ARGUMENT, "%s: null norm or modulation vector", stage);
  if (!aligned(norm_scale, 16) || !aligned(mod_scale, 16) || !aligned(mod_shift, 16))
    return fail(K2W8_INVALID_ARGUMENT, "%s: norm and modulation vectors must be 16-byte aligned", stage);
  if (!(cfg->eps >= 0.0f)) return fail(K2W8_INVALID_ARGUMENT, "%s: eps must be >= 0", stage);
  if ((rc = ensure_configured(stage)) != K2W8_OK) return rc;
  k2w8::PrepareLaunch p;
  p.h = h;
  p.norm_scale = norm_scale;
  p.mod_scale = mod_scale;
  p.mod_shift = mod_shift;
  p.q = q;
  p.q_scale = q_scale;
  p.width = cfg->width;
  p.out_stride = cfg->out_stride;
  p.eps = cfg->eps;
  hipError_t e = k2w8::launch_prepare(0, static_cast<hipStream_t>(stream), tokens, p);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

int k2w8_prepare_plain_i8(void *stream, const k2w8_prepare_plain_cfg *cfg, int64_t tokens,
                          const void *h, int8_t *q, float *q_scale) {
  const char *stage = "prepare_plain_i8";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  int rc = check_prepare(stage, tokens, cfg->width, cfg->out_stride, h, q, q_scale);
  if (rc != K2W8_OK) return rc;
  if ((rc = ensure_configured(stage)) != K2W8_OK) return rc;
  k2w8::PrepareLaunch p;
  p.h = h;
  p.q = q;
  p.q_scale = q_scale;
  p.width = cfg->width;
  p.out_stride = cfg->out_stride;
  hipError_t e = k2w8::launch_prepare(1, static_cast<hipStream_t>(stream), tokens, p);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

int k2w8_prepare_gated_i8(void *stream, const k2w8_prepare_gated_cfg *cfg, int64_t tokens,
                          const void *attn, const void *gate, int8_t *q, float *q_scale) {
  const char *stage = "prepare_gated_i8";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  int rc = check_prepare(stage, tokens, cfg->width, cfg->out_stride, attn, q, q_scale);
  if (rc != K2W8_OK) return rc;
  if (!gate) return fail(K2W8_INVALID_ARGUMENT, "%s: null gate", stage);
  if (cfg->gate_stride < cfg->width || cfg->gate_stride > 65536 || cfg->gate_stride % 8 != 0)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: gate_stride must be a multiple of 8 in width..65536, got %lld", stage,
                (long long)cfg->gate_stride);
  if (!aligned(gate, 16)) return fail(K2W8_INVALID_ARGUMENT, "%s: gate must be 16-byte aligned", stage);
  if ((rc = ensure_configured(stage)) != K2W8_OK) return rc;
  k2w8::PrepareLaunch p;
  p.h = attn;
  p.gate = gate;
  p.q = q;
  p.q_scale = q_scale;
  p.width = cfg->width;
  p.out_stride = cfg->out_stride;
  p.gate_stride = cfg->gate_stride;
  hipError_t e = k2w8::launch_prepare(2, static_cast<hipStream_t>(stream), tokens, p);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

int k2w8_gemm_i8(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                 const int8_t *w, const float *scale, const float *a_scale, void *c) {
  return run_gemm("gemm_i8", k2w8::kEpiPlain, stream, cfg, m, a, w, scale, a_scale, c, nullptr,
                  nullptr);
}

int k2w8_gemm_i8_resid(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                       const int8_t *w, const float *scale, const float *a_scale, void *c,
                       const float *gate) {
  return run_gemm("gemm_i8_resid", k2w8::kEpiResid, stream, cfg, m, a, w, scale, a_scale, c,
                  gate, nullptr);
}

int k2w8_gemm_i8_resid_256x256(void *stream, const k2w8_gemm_cfg *cfg, int64_t m,
                               const int8_t *a, const int8_t *w, const float *scale,
                               const float *a_scale, void *c, const float *gate) {
  return run_gemm("gemm_i8_resid_256x256", k2w8::kEpiResid, stream, cfg, m, a, w, scale, a_scale,
                  c, gate, nullptr);
}

int k2w8_gemm_i8_swiglu(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                        const int8_t *w, const float *scale, const float *a_scale, void *c) {
  return run_gemm("gemm_i8_swiglu", k2w8::kEpiSwiglu, stream, cfg, m, a, w, scale, a_scale, c,
                  nullptr, nullptr);
}

int k2w8_gemm_i8_bias(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                      const int8_t *w, const float *scale, const float *a_scale, const void *bias,
                      void *c) {
  return run_gemm("gemm_i8_bias", k2w8::kEpiBias, stream, cfg, m, a, w, scale, a_scale, c,
                  nullptr, bias);
}

int k2w8_gemm_i8_acc(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                     const int8_t *w, int32_t *acc) {
  // This epilogue reads no scales; the int32 output stands in for them in validation
  // and the kernel never dereferences them.
  const float *unused = reinterpret_cast<const float *>(acc);
  return run_gemm("gemm_i8_acc", k2w8::kEpiAcc, stream, cfg, m, a, w, unused, unused, acc,
                  nullptr, nullptr);
}

int k2w8_lora_transport(void *stream, int direction, int64_t count, const void *x, void *out) {
  const char *stage = "lora_transport";
  if (direction != 1 && direction != 2)
    return fail(K2W8_INVALID_ARGUMENT, "%s: direction must be 1 (bf16 -> f16) or 2 (f16 -> bf16), got %d",
                stage, direction);
  // kernels/native/lora_transport.loom:13
  if (count < 1 || count >= (int64_t(1) << 30))
    return fail(K2W8_INVALID_ARGUMENT, "%s: count must be 1..2^30-1, got %lld", stage,
                (long long)count);
  if (!x || !out) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(x, 16) || !aligned(out, 16))
    return fail(K2W8_INVALID_ARGUMENT, "%s: x and out must be 16-byte aligned", stage);
  hipError_t e = k2w8::launch_transport(direction, static_cast<hipStream_t>(stream), count, x, out);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

// src/training/quantized.rs:51-112
int k2w8_quantized_forward(void *stream, const k2w8_quantized_cfg *cfg, int64_t rows,
                           const void *x, const int8_t *weight, const float *scales,
                           void *transport, int8_t *quantized, float *q_scales, void *out_f16,
                           void *out) {
  const char *stage = "quantized_forward";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  if (rows < 1 || rows * cfg->inputs >= (int64_t(1) << 30) ||
      rows * cfg->outputs >= (int64_t(1) << 30))
    return fail(K2W8_INVALID_ARGUMENT, "%s: rows * inputs and rows * outputs must be below 2^30",
                stage);
  int rc = k2w8_lora_transport(stream, 1, rows * cfg->inputs, x, transport);
  if (rc != K2W8_OK) return rc;
  const k2w8_prepare_plain_cfg prep = {cfg->inputs, cfg->pitch};
  rc = k2w8_prepare_plain_i8(stream, &prep, rows, transport, quantized, q_scales);
  if (rc != K2W8_OK) return rc;
  const k2w8_gemm_cfg gemm = {cfg->inputs, cfg->outputs, cfg->pitch, k2w8_shape_gemm_m_group(), 0};
  rc = k2w8_gemm_i8(stream, &gemm, rows, quantized, weight, scales, q_scales, out_f16);
  if (rc != K2W8_OK) return rc;
  return k2w8_lora_transport(stream, 2, rows * cfg->outputs, out_f16, out);
}

// src/kernels/shape.rs:105-107
int64_t k2w8_shape_gemm_pitch(int64_t k) { return (k % 8192 == 0) ? k + 64 : k; }

// src/kernels/shape.rs:12-16
int64_t k2w8_shape_capacity(int64_t tokens) {
  int64_t tiles = (tokens + 16 + 31) / 32 * 32;
  int64_t blocks = (tokens + 63) / 64 * 64;
  return tiles > blocks ? tiles : blocks;
}

// src/kernels/shape.rs:110-112
int64_t k2w8_shape_gemm_grid_rows(int64_t tokens) { return (tokens + 255) / 256; }

// src/kernels/shape.rs:97-99
int k2w8_shape_gemm_schedule_rows(int64_t tokens) { return tokens >= 4096 ? 1 : 0; }

int64_t k2w8_shape_gemm_rows(void) { return 256; }
int64_t k2w8_shape_gemm_m_group(void) { return 4; }
int64_t k2w8_shape_tokens_min(void) { return 16; }
int64_t k2w8_shape_tokens_max(void) { return 16896; }

}  // extern "C"
