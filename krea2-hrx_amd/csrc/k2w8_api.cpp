// The C ABI (include/krea2_w8a8.h): argument validation mirroring the reference's
// `config.decl` constraints, the launch-shape rules of src/kernels/shape.rs, and
// the three-way error split of src/error.rs:11-29.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "krea2_w8a8.h"
#include "k2w8_internal.hpp"
#include "k2w8_gemm_plan.hpp"

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

// Large dynamic LDS is enabled per kernel, once per device (the first call there).
int ensure_configured(const char *stage) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static bool done[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(K2W8_RUNTIME, "%s: the current device: %s", stage, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(K2W8_RUNTIME, "%s: device %d is past the library's %d", stage, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (done[dev]) return K2W8_OK;
  if ((e = k2w8::configure_prepare_lds()) != hipSuccess)
    return fail(K2W8_RUNTIME, "%s: enabling the prepare kernels' LDS: %s", stage, hipGetErrorString(e));
  if ((e = k2w8::configure_gemm_lds()) != hipSuccess)
    return fail(K2W8_RUNTIME, "%s: enabling the GEMM kernels' LDS: %s", stage, hipGetErrorString(e));
  if ((e = k2w8::configure_fused_lds()) != hipSuccess)
    return fail(K2W8_RUNTIME, "%s: enabling the one-launch kernels' LDS: %s", stage, hipGetErrorString(e));
  done[dev] = true;
  return K2W8_OK;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Token bound of the prepares and GEMMs (kernels/prepare_norm_i8.loom:56, gemm m range).
constexpr int64_t kMaxTokens = 1 << 20;

int check_prepare_shape(const char *stage, int64_t width, int64_t out_stride) {
  if (width < 256 || width > 32768 || width % 256 != 0)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: width must be a multiple of 256 in 256..32768, got %lld", stage,
                (long long)width);
  if (out_stride < width || out_stride > 65536 || out_stride % 64 != 0)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: out_stride must be a multiple of 64 in width..65536, got %lld", stage,
                (long long)out_stride);
  return K2W8_OK;
}

int check_prepare(const char *stage, int64_t tokens, int64_t width, int64_t out_stride,
                  const void *h, const int8_t *q, const float *q_scale) {
  if (tokens < 1 || tokens > kMaxTokens)
    return fail(K2W8_INVALID_ARGUMENT, "%s: tokens must be 1..%lld, got %lld", stage,
                (long long)kMaxTokens, (long long)tokens);
  const int rc = check_prepare_shape(stage, width, out_stride);
  if (rc != K2W8_OK) return rc;
  if (!h || !q || !q_scale) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(h, 16) || !aligned(q, 16) || !aligned(q_scale, 4))
    return fail(K2W8_INVALID_ARGUMENT, "%s: h and q must be 16-byte aligned", stage);
  return K2W8_OK;
}

// The norm prepare's vectors (kernels/prepare_norm_i8.loom:22) and eps.
int check_norm_vectors(const char *stage, const float *norm_scale, const float *mod_scale,
                       const float *mod_shift, float eps) {
  if (!norm_scale || !mod_scale || !mod_shift)
    return fail(K2W8_INVALID_ARGUMENT, "%s: null norm or modulation vector", stage);
  if (!aligned(norm_scale, 16) || !aligned(mod_scale, 16) || !aligned(mod_shift, 16))
    return fail(K2W8_INVALID_ARGUMENT, "%s: norm and modulation vectors must be 16-byte aligned", stage);
  if (!(eps >= 0.0f)) return fail(K2W8_INVALID_ARGUMENT, "%s: eps must be >= 0", stage);
  return K2W8_OK;
}

// The gated prepare's gate operand and its row stride (kernels/prepare_gated_i8.loom:16).
int check_gate_input(const char *stage, const void *gate, int64_t width, int64_t gate_stride) {
  if (!gate) return fail(K2W8_INVALID_ARGUMENT, "%s: null gate", stage);
  if (gate_stride < width || gate_stride > 65536 || gate_stride % 8 != 0)
    return fail(K2W8_INVALID_ARGUMENT, "%s: gate_stride must be a multiple of 8 in width..65536, got %lld",
                stage, (long long)gate_stride);
  if (!aligned(gate, 16)) return fail(K2W8_INVALID_ARGUMENT, "%s: gate must be 16-byte aligned", stage);
  return K2W8_OK;
}

// The gated prepare's sigmoid table is uploaded on the first call on a device, which
// must not happen inside a stream capture.
int gated_ready(const char *stage, hipStream_t stream) {
  const hipError_t e = k2w8::prepare_gated_ready(stream);
  if (e == hipErrorStreamCaptureUnsupported)
    return fail(K2W8_RUNTIME, "%s: the first gated call on a device must not be inside a stream capture "
                "(k2w8_prime_launches sets the device up beforehand)", stage);
  if (e != hipSuccess) return runtime(stage, e);
  return K2W8_OK;
}

int check_gemm_cfg(const char *stage, const k2w8_gemm_cfg *cfg) {
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
  if (cfg->schedule_rows < 0 || cfg->schedule_rows > 1)
    return fail(K2W8_INVALID_ARGUMENT, "%s: schedule_rows must be 0 or 1, got %lld", stage,
                (long long)cfg->schedule_rows);
  return K2W8_OK;
}

int check_gemm(const char *stage, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
               const int8_t *w, const float *scale, const float *a_scale, const void *c) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  int rc = check_gemm_cfg(stage, cfg);
  if (rc != K2W8_OK) return rc;
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
             const float *gate, const void *bias, const k2w8::Workspace *fixed = nullptr) {
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
  l.workspace = fixed;
  l.workspace_required = fixed != nullptr;
  hipError_t e = k2w8::launch_gemm(epi, static_cast<hipStream_t>(stream), l);
  if (e == hipErrorInvalidValue && fixed)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: m=%lld x n_size=%lld splits K and needs %lld bytes of scratch for two int32 "
                "slices; the static scratch holds %lld", stage, (long long)m,
                (long long)cfg->n_size, (long long)(2 * m * cfg->n_size * 4),
                (long long)fixed->bytes);
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
int k2w8_prime_launches(void *stream) {
  int rc = ensure_configured("blocks_record");
  if (rc != K2W8_OK) return rc;
  (void)k2w8::device_cus();
  const hipError_t e = k2w8::prepare_gated_ready(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return runtime("blocks_record: the gated prepare's sigmoid table", e);
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
  if ((rc = check_norm_vectors(stage, norm_scale, mod_scale, mod_shift, cfg->eps)) != K2W8_OK) return rc;
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

// One-call prepare -> GEMM: a prepare (kind 0 norm, 1 plain, 2 gated) and the GEMM that
// reads its q / q_scale, with the given epilogue. Both halves are validated as their
// own entry points validate them, before either launches.
struct LinearPrepare {
  int kind;
  int64_t width, out_stride, gate_stride;
  float eps;
  const void *h, *gate_in;
  const float *norm_scale, *mod_scale, *mod_shift;
};

static int run_linear(const char *stage, const LinearPrepare &lp, int epi, void *stream,
                      const k2w8_gemm_cfg *gcfg, int64_t tokens, int8_t *q, float *q_scale,
                      const int8_t *w, const float *scale, void *c, const float *gate) {
  if (!gcfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  int rc = check_prepare(stage, tokens, lp.width, lp.out_stride, lp.h, q, q_scale);
  if (rc != K2W8_OK) return rc;
  if ((rc = check_gemm(stage, gcfg, tokens, q, w, scale, q_scale, c)) != K2W8_OK) return rc;
  if (gcfg->k_size != lp.width || gcfg->k_stride != lp.out_stride)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: the GEMM's k_size and k_stride must be the prepare's width and out_stride", stage);
  if (lp.kind == 0 &&
      (rc = check_norm_vectors(stage, lp.norm_scale, lp.mod_scale, lp.mod_shift, lp.eps)) != K2W8_OK)
    return rc;
  if (lp.kind == 2 && (rc = check_gate_input(stage, lp.gate_in, lp.width, lp.gate_stride)) != K2W8_OK)
    return rc;
  if (epi == k2w8::kEpiResid && !gate) return fail(K2W8_INVALID_ARGUMENT, "%s: null residual gate", stage);
  if (gate && !aligned(gate, 16))
    return fail(K2W8_INVALID_ARGUMENT, "%s: the residual gate must be 16-byte aligned", stage);
  if ((rc = ensure_configured(stage)) != K2W8_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (lp.kind == 2 && (rc = gated_ready(stage, s)) != K2W8_OK) return rc;
  k2w8::PrepareLaunch p;
  p.h = lp.h;
  p.gate = lp.gate_in;
  p.norm_scale = lp.norm_scale;
  p.mod_scale = lp.mod_scale;
  p.mod_shift = lp.mod_shift;
  p.q = q;
  p.q_scale = q_scale;
  p.width = lp.width;
  p.out_stride = lp.out_stride;
  p.gate_stride = lp.gate_stride;
  p.eps = lp.eps;
  k2w8::GemmLaunch l;
  l.a = q;
  l.w = w;
  l.w_scale = scale;
  l.a_scale = q_scale;
  l.c = c;
  l.gate = gate;
  l.m = tokens;
  l.n = gcfg->n_size;
  l.k = gcfg->k_size;
  l.lda = gcfg->k_stride;
  l.m_group = (int)gcfg->m_group;
  // Two launches by default: the one-launch form (norm or plain prepare, plain
  // epilogue) measured slower (configs[1] 135 -> 148 us: its prepare phase runs at one
  // workgroup per CU, and the grid barrier's agent-scope release and acquire write
  // back and invalidate each XCD's L2). Setting K2W8_LINEAR_ONE_LAUNCH=1 selects it
  // (read on every call).
  const char *one = getenv("K2W8_LINEAR_ONE_LAUNCH");
  hipError_t e = (one && one[0] == '1' && lp.kind != 2 && epi == k2w8::kEpiPlain)
                     ? k2w8::launch_prepare_gemm(lp.kind, s, tokens, p, l)
                     : hipErrorNotSupported;
  if (e == hipErrorNotSupported) {
    e = k2w8::launch_prepare(lp.kind, s, tokens, p);
    if (e == hipSuccess) e = k2w8::launch_gemm(epi, s, l);
  }
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

static LinearPrepare norm_prepare(const k2w8_prepare_norm_cfg *cfg, const void *h, const float *ns,
                                  const float *ms, const float *sh) {
  return LinearPrepare{0, cfg->width, cfg->out_stride, 0, cfg->eps, h, nullptr, ns, ms, sh};
}
static LinearPrepare plain_prepare(const k2w8_prepare_plain_cfg *cfg, const void *h) {
  return LinearPrepare{1, cfg->width, cfg->out_stride, 0, 0.0f, h, nullptr, nullptr, nullptr, nullptr};
}

int k2w8_linear_norm_i8(void *stream, const k2w8_prepare_norm_cfg *cfg, const k2w8_gemm_cfg *gemm,
                        int64_t tokens, const void *h, const float *norm_scale,
                        const float *mod_scale, const float *mod_shift, int8_t *q,
                        float *q_scale, const int8_t *w, const float *scale, void *c) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "linear_norm_i8: null configuration");
  return run_linear("linear_norm_i8", norm_prepare(cfg, h, norm_scale, mod_scale, mod_shift), k2w8::kEpiPlain,
                    stream, gemm, tokens, q, q_scale, w, scale, c, nullptr);
}

int k2w8_linear_plain_i8(void *stream, const k2w8_prepare_plain_cfg *cfg, const k2w8_gemm_cfg *gemm,
                         int64_t tokens, const void *h, int8_t *q, float *q_scale,
                         const int8_t *w, const float *scale, void *c) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "linear_plain_i8: null configuration");
  return run_linear("linear_plain_i8", plain_prepare(cfg, h), k2w8::kEpiPlain, stream, gemm, tokens, q,
                    q_scale, w, scale, c, nullptr);
}

int k2w8_linear_gated_resid_i8(void *stream, const k2w8_prepare_gated_cfg *cfg, const k2w8_gemm_cfg *gemm,
                               int64_t tokens, const void *attn, const void *gate_in, int8_t *q,
                               float *q_scale, const int8_t *w, const float *scale, void *x,
                               const float *gate) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "linear_gated_resid_i8: null configuration");
  const LinearPrepare lp{2, cfg->width, cfg->out_stride, cfg->gate_stride, 0.0f, attn, gate_in,
                         nullptr, nullptr, nullptr};
  return run_linear("linear_gated_resid_i8", lp, k2w8::kEpiResid, stream, gemm, tokens, q, q_scale, w, scale,
                    x, gate);
}

int k2w8_linear_norm_swiglu_i8(void *stream, const k2w8_prepare_norm_cfg *cfg, const k2w8_gemm_cfg *gemm,
                               int64_t tokens, const void *h, const float *norm_scale,
                               const float *mod_scale, const float *mod_shift, int8_t *q,
                               float *q_scale, const int8_t *w, const float *scale, void *c) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "linear_norm_swiglu_i8: null configuration");
  return run_linear("linear_norm_swiglu_i8", norm_prepare(cfg, h, norm_scale, mod_scale, mod_shift),
                    k2w8::kEpiSwiglu, stream, gemm, tokens, q, q_scale, w, scale, c, nullptr);
}

int k2w8_linear_plain_resid_i8(void *stream, const k2w8_prepare_plain_cfg *cfg, const k2w8_gemm_cfg *gemm,
                               int64_t tokens, const void *h, int8_t *q, float *q_scale,
                               const int8_t *w, const float *scale, void *x, const float *gate) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "linear_plain_resid_i8: null configuration");
  return run_linear("linear_plain_resid_i8", plain_prepare(cfg, h), k2w8::kEpiResid, stream, gemm, tokens,
                    q, q_scale, w, scale, x, gate);
}

int k2w8_prepare_gated_i8(void *stream, const k2w8_prepare_gated_cfg *cfg, int64_t tokens,
                          const void *attn, const void *gate, int8_t *q, float *q_scale) {
  const char *stage = "prepare_gated_i8";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  int rc = check_prepare(stage, tokens, cfg->width, cfg->out_stride, attn, q, q_scale);
  if (rc != K2W8_OK) return rc;
  if ((rc = check_gate_input(stage, gate, cfg->width, cfg->gate_stride)) != K2W8_OK) return rc;
  if ((rc = ensure_configured(stage)) != K2W8_OK) return rc;
  if ((rc = gated_ready(stage, static_cast<hipStream_t>(stream))) != K2W8_OK) return rc;
  k2w8::PrepareLaunch p;
  p.h = attn;
  p.gate = gate;
  p.q = q;
  p.q_scale = q_scale;
  p.width = cfg->width;
  p.out_stride = cfg->out_stride;
  p.gate_stride = cfg->gate_stride;
  const hipError_t e = k2w8::launch_prepare(2, static_cast<hipStream_t>(stream), tokens, p);
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

int k2w8_gemm_i8_noalloc(void *stream, const k2w8_gemm_cfg *cfg, int64_t m, const int8_t *a,
                         const int8_t *w, const float *scale, const float *a_scale, void *c) {
  const char *stage = "gemm_i8_noalloc";
  int rc = check_gemm(stage, cfg, m, a, w, scale, a_scale, c);
  if (rc != K2W8_OK) return rc;
  hipError_t e = hipSuccess;
  const k2w8::Workspace scratch = k2w8::splitk_static_scratch(&e);
  if (e != hipSuccess) return runtime("gemm_i8_noalloc: the static scratch's set-up", e);
  // Only a split-K launch touches the scratch: those calls are ordered on the device.
  const int64_t cus = k2w8::device_cus();
  k2w8::GemmLaunch l;
  l.m = m;
  l.n = cfg->n_size;
  l.k = cfg->k_size;
  const bool splits = !k2w8::gemm_streams(k2w8::kEpiPlain, l, cus) &&
                      k2w8::plan_tiles(l.m, l.n, l.k, cus).tile == k2w8::GemmTile::kSplit &&
                      k2w8::splitk_steps(l.m, l.n, l.k, cus, scratch.bytes) > 0;
  if (!splits)
    return run_gemm(stage, k2w8::kEpiPlain, stream, cfg, m, a, w, scale, a_scale, c, nullptr, nullptr,
                    &scratch);
  rc = K2W8_OK;
  e = k2w8::splitk_static_ordered(static_cast<hipStream_t>(stream), [&]() {
    rc = run_gemm(stage, k2w8::kEpiPlain, stream, cfg, m, a, w, scale, a_scale, c, nullptr, nullptr, &scratch);
    return hipSuccess;
  });
  if (rc != K2W8_OK) return rc;
  if (e != hipSuccess) return runtime("gemm_i8_noalloc: ordering the static scratch's users", e);
  return ok();
}

int k2w8_gemm_choose(int32_t epilogue, int64_t m, const k2w8_gemm_cfg *cfg, int64_t cus,
                     int64_t workspace_bytes, int32_t workspace_required, k2w8_gemm_choice *out) {
  const char *stage = "gemm_choose";
  if (!cfg || !out) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration or output", stage);
  int rc = check_gemm_cfg(stage, cfg);
  if (rc != K2W8_OK) return rc;
  if (epilogue < 0 || epilogue > k2w8::kEpiAcc)
    return fail(K2W8_INVALID_ARGUMENT, "%s: epilogue must be 0..4, got %d", stage, (int)epilogue);
  if (m < 1 || m > 16777216)
    return fail(K2W8_INVALID_ARGUMENT, "%s: m must be 1..16777216, got %lld", stage, (long long)m);
  if (cus < 1 || cus > 4096 || workspace_bytes < 0)
    return fail(K2W8_INVALID_ARGUMENT, "%s: cus must be 1..4096 and workspace_bytes >= 0", stage);
  k2w8::GemmLaunch l;
  l.m = m;
  l.n = cfg->n_size;
  l.k = cfg->k_size;
  l.lda = cfg->k_stride;
  *out = k2w8_gemm_choice{};
  if (k2w8::gemm_streams(epilogue, l, cus)) return ok();  // kernel 0
  using k2w8::GemmTile;
  const k2w8::TilePlan plan = k2w8::plan_tiles(l.m, l.n, l.k, cus);
  struct Shape {
    int32_t m, n, stages;
  };
  static const Shape kShapes[] = {{256, 256, 2}, {256, 192, 2}, {256, 128, 2}, {256, 128, 3},
                                  {128, 128, 2}, {128, 64, 3},  {64, 64, 4},   {128, 128, 3}};
  int tile = (int)plan.tile;
  out->kernel = plan.n_big > 0 ? 2 : 1;
  out->n_big = plan.n_big;
  if (plan.tile == GemmTile::kSplit) {
    if (workspace_required && k2w8::splitk_refused(l.m, l.n, l.k, cus, (size_t)workspace_bytes)) {
      out->kernel = -1;  // the entry point refuses the shape with INVALID_ARGUMENT
      return ok();
    }
    const int per = k2w8::splitk_steps(l.m, l.n, l.k, cus, (size_t)workspace_bytes);
    if (per > 0) {
      out->kernel = 3;
      out->split_steps = per;
      out->splits = (int32_t)((l.k / 128 + per - 1) / per);
    } else {
      tile = (int)GemmTile::k64x64;  // no split without room for two slices
    }
  }
  out->tile_m = kShapes[tile].m;
  out->tile_n = kShapes[tile].n;
  out->stages = kShapes[tile].stages;
  return ok();
}

int k2w8_gemm_set_workspace(void *stream, void *workspace, int64_t bytes) {
  if (workspace && (bytes < 256 || !aligned(workspace, 256)))
    return fail(K2W8_INVALID_ARGUMENT,
                "gemm_set_workspace: workspace must be 256-byte aligned and at least 256 bytes, "
                "got %lld bytes", (long long)bytes);
  hipError_t e = k2w8::splitk_register(static_cast<hipStream_t>(stream), workspace,
                                       workspace ? (size_t)bytes : 0);
  if (e != hipSuccess) return runtime("gemm_set_workspace", e);
  return ok();
}

int64_t k2w8_gemm_workspace_bytes(void) { return (int64_t)k2w8::splitk_workspace_bytes(); }

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

int k2w8_sigmoid_f32(void *stream, int64_t count, const float *x, float *out) {
  const char *stage = "sigmoid_f32";
  if (count < 1 || count >= (int64_t(1) << 32))
    return fail(K2W8_INVALID_ARGUMENT, "%s: count must be 1..2^32-1, got %lld", stage,
                (long long)count);
  if (!x || !out) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(x, 4) || !aligned(out, 4))
    return fail(K2W8_INVALID_ARGUMENT, "%s: x and out must be 4-byte aligned", stage);
  hipError_t e = k2w8::launch_sigmoid(static_cast<hipStream_t>(stream), count, x, out);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

// kernels/rope_qknorm_f16.loom:12-20, 22-159
int k2w8_rope_qknorm_f16(void *stream, const k2w8_rope_qknorm_cfg *cfg, int64_t tokens,
                         const void *qkv, const float *q_scale, const float *k_scale,
                         const float *cos, const float *sin, void *q_out, void *k_out,
                         void *v_out) {
  const char *stage = "rope_qknorm_f16";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  if (cfg->row_stride < 128 || cfg->row_stride > 65536 || cfg->row_stride % 128)
    return fail(K2W8_INVALID_ARGUMENT, "%s: row_stride must be a multiple of 128 in 128..65536, got %lld",
                stage, (long long)cfg->row_stride);
  if (cfg->q_heads < 1 || cfg->q_heads > 256 || cfg->kv_heads < 1 || cfg->kv_heads > 256)
    return fail(K2W8_INVALID_ARGUMENT, "%s: q_heads and kv_heads must be in 1..256", stage);
  if (cfg->k_offset < 128 || cfg->k_offset > 65536 || cfg->k_offset % 128)
    return fail(K2W8_INVALID_ARGUMENT, "%s: k_offset must be a multiple of 128 in 128..65536, got %lld",
                stage, (long long)cfg->k_offset);
  if (cfg->q_heads * 128 > cfg->row_stride || cfg->k_offset + 2 * cfg->kv_heads * 128 > cfg->row_stride)
    return fail(K2W8_INVALID_ARGUMENT, "%s: q heads and k_offset + 2 * kv_heads * 128 must fit row_stride",
                stage);
  if (!(cfg->eps >= 0.0f)) return fail(K2W8_INVALID_ARGUMENT, "%s: eps must be >= 0", stage);
  if (tokens < 1 || tokens > (int64_t(1) << 20))
    return fail(K2W8_INVALID_ARGUMENT, "%s: tokens must be in 1..2^20, got %lld", stage, (long long)tokens);
  if (!qkv || !q_scale || !k_scale || !cos || !sin || !q_out || !k_out || !v_out)
    return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  for (const void *p : {qkv, (const void *)q_scale, (const void *)k_scale, (const void *)cos,
                        (const void *)sin, (const void *)q_out, (const void *)k_out, (const void *)v_out})
    if (!aligned(p, 16)) return fail(K2W8_INVALID_ARGUMENT, "%s: every buffer must be 16-byte aligned", stage);
  k2w8::RopeLaunch l;
  l.qkv = qkv;
  l.q_scale = q_scale;
  l.k_scale = k_scale;
  l.cos = cos;
  l.sin = sin;
  l.q_out = q_out;
  l.k_out = k_out;
  l.v_out = v_out;
  l.tokens = tokens;
  l.row_stride = cfg->row_stride;
  l.q_heads = cfg->q_heads;
  l.kv_heads = cfg->kv_heads;
  l.k_offset = cfg->k_offset;
  l.eps = cfg->eps;
  hipError_t e = k2w8::launch_rope_qknorm(static_cast<hipStream_t>(stream), l);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

// kernels/native/v_transpose.loom:7-9, 11-90
int k2w8_v_transpose(void *stream, const k2w8_v_transpose_cfg *cfg, int64_t rows, const void *x,
                     void *out) {
  const char *stage = "v_transpose";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  if (cfg->width < 32 || cfg->width > 65536 || cfg->width % 32)
    return fail(K2W8_INVALID_ARGUMENT, "%s: width must be a multiple of 32 in 32..65536, got %lld", stage,
                (long long)cfg->width);
  if (cfg->row_capacity < 32 || cfg->row_capacity > (int64_t(1) << 20) || cfg->row_capacity % 32)
    return fail(K2W8_INVALID_ARGUMENT, "%s: row_capacity must be a multiple of 32 in 32..2^20, got %lld",
                stage, (long long)cfg->row_capacity);
  if (rows < 1 || rows > cfg->row_capacity)
    return fail(K2W8_INVALID_ARGUMENT, "%s: rows must be in 1..row_capacity, got %lld", stage,
                (long long)rows);
  if (!x || !out) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(x, 16) || !aligned(out, 16))
    return fail(K2W8_INVALID_ARGUMENT, "%s: x and out must be 16-byte aligned", stage);
  hipError_t e = k2w8::launch_v_transpose(static_cast<hipStream_t>(stream), rows, cfg->width,
                                          cfg->row_capacity, x, out);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

// kernels/attention_gqa_lds_f16_wmma.loom:18-28, 30-380
int k2w8_attention_f16(void *stream, const k2w8_attention_cfg *cfg, int64_t token_count,
                       int64_t kv_head_count, const void *q, const void *k, const void *v,
                       void *out) {
  return k2w8_attention_f16_grouped(stream, cfg, token_count, kv_head_count, 4, q, k, v, out);
}

int k2w8_attention_f16_grouped(void *stream, const k2w8_attention_cfg *cfg, int64_t token_count,
                               int64_t kv_head_count, int64_t group, const void *q, const void *k,
                               const void *v, void *out) {
  const char *stage = "attention_f16";
  if (group != 1 && group != 2 && group != 4)
    return fail(K2W8_INVALID_ARGUMENT, "%s: group must be 1, 2 or 4, got %lld", stage, (long long)group);
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  for (int64_t s : {cfg->q_stride, cfg->kv_stride, cfg->out_stride})
    if (s < 128 || s > 32768 || s % 128)
      return fail(K2W8_INVALID_ARGUMENT, "%s: strides must be multiples of 128 in 128..32768, got %lld",
                  stage, (long long)s);
  if (cfg->tokens < 16 || cfg->tokens > 65536)
    return fail(K2W8_INVALID_ARGUMENT, "%s: tokens must be in 16..65536, got %lld", stage,
                (long long)cfg->tokens);
  if (cfg->token_capacity % 16 || cfg->token_capacity > (int64_t(1) << 20) ||
      cfg->token_capacity < cfg->tokens + 16)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: token_capacity must be a multiple of 16, >= tokens + 16 and <= 2^20, got %lld", stage,
                (long long)cfg->token_capacity);
  if (!(cfg->scale > 0.0f) || !(cfg->scale < 1e30f))
    return fail(K2W8_INVALID_ARGUMENT, "%s: scale must be positive and finite", stage);
  if (token_count < 1 || token_count > cfg->token_capacity)
    return fail(K2W8_INVALID_ARGUMENT, "%s: token_count must be in 1..token_capacity, got %lld", stage,
                (long long)token_count);
  if (kv_head_count < 1 || kv_head_count * 128 > cfg->kv_stride ||
      group * kv_head_count * 128 > cfg->q_stride || group * kv_head_count * 128 > cfg->out_stride)
    return fail(K2W8_INVALID_ARGUMENT,
                "%s: kv_head_count must be >= 1 with kv_head_count*128 <= kv_stride and "
                "group*kv_head_count*128 <= q_stride, out_stride (got %lld)",
                stage, (long long)kv_head_count);
  if (!q || !k || !v || !out) return fail(K2W8_INVALID_ARGUMENT, "%s: null buffer", stage);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
    return fail(K2W8_INVALID_ARGUMENT, "%s: q, k, v and out must be 16-byte aligned", stage);
  k2w8::AttentionLaunch l;
  l.q = q;
  l.k = k;
  l.vt = v;
  l.out = out;
  l.tokens = cfg->tokens;
  l.rows_out = token_count < cfg->tokens ? token_count : cfg->tokens;
  l.capacity = cfg->token_capacity;
  l.q_stride = cfg->q_stride;
  l.kv_stride = cfg->kv_stride;
  l.out_stride = cfg->out_stride;
  l.kv_heads = kv_head_count;
  l.group = group;
  l.scale = cfg->scale;
  hipError_t e = k2w8::launch_attention(static_cast<hipStream_t>(stream), l);
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
// Measurement aid (no reference counterpart): the MFMA-only INT8 rate, k2w8_probe.hip.
int k2w8_probe_mfma_i8(void *stream, int64_t blocks, int64_t iters, int32_t random, uint32_t seed,
                       int32_t *out) {
  const char *stage = "probe_mfma_i8";
  if (blocks < 1 || blocks > 65536 || iters < 1 || iters > (int64_t(1) << 24))
    return fail(K2W8_INVALID_ARGUMENT, "%s: blocks must be 1..65536 and iters 1..2^24", stage);
  if (!out || !aligned(out, 4)) return fail(K2W8_INVALID_ARGUMENT, "%s: null or misaligned out", stage);
  const hipError_t e = k2w8::launch_probe_mfma(static_cast<hipStream_t>(stream), blocks, iters, random ? 1 : 0,
                                               seed, out);
  if (e != hipSuccess) return runtime(stage, e);
  return ok();
}

// Configuration checks alone, as the reference's config.decl ranges constrain each
// kernel's specialisation (kernels/gemm_i8_256.loom:14-22,
// kernels/prepare_norm_i8.loom:11-16, kernels/prepare_plain_i8.loom:10-13,
// kernels/prepare_gated_i8.loom:11-16): a caller can check a configuration once, before
// it records or launches anything. The entry points run the same checks.
int k2w8_validate_gemm_cfg(const k2w8_gemm_cfg *cfg) {
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "validate_gemm_cfg: null configuration");
  const int rc = check_gemm_cfg("validate_gemm_cfg", cfg);
  return rc != K2W8_OK ? rc : ok();
}

int k2w8_validate_prepare_norm_cfg(const k2w8_prepare_norm_cfg *cfg) {
  const char *stage = "validate_prepare_norm_cfg";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  const int rc = check_prepare_shape(stage, cfg->width, cfg->out_stride);
  if (rc != K2W8_OK) return rc;
  if (!(cfg->eps >= 0.0f)) return fail(K2W8_INVALID_ARGUMENT, "%s: eps must be >= 0", stage);
  return ok();
}

int k2w8_validate_prepare_plain_cfg(const k2w8_prepare_plain_cfg *cfg) {
  const char *stage = "validate_prepare_plain_cfg";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  const int rc = check_prepare_shape(stage, cfg->width, cfg->out_stride);
  return rc != K2W8_OK ? rc : ok();
}

int k2w8_validate_prepare_gated_cfg(const k2w8_prepare_gated_cfg *cfg) {
  const char *stage = "validate_prepare_gated_cfg";
  if (!cfg) return fail(K2W8_INVALID_ARGUMENT, "%s: null configuration", stage);
  const int rc = check_prepare_shape(stage, cfg->width, cfg->out_stride);
  if (rc != K2W8_OK) return rc;
  if (cfg->gate_stride < cfg->width || cfg->gate_stride > 65536 || cfg->gate_stride % 8 != 0)
    return fail(K2W8_INVALID_ARGUMENT, "%s: gate_stride must be a multiple of 8 in width..65536, got %lld",
                stage, (long long)cfg->gate_stride);
  return ok();
}

// The shape rules take the reference's usize sizes; here they answer for 0..2^40 and
// return -1 outside it (a negative size, or one whose arithmetic would overflow).
constexpr int64_t kShapeDomain = int64_t(1) << 40;

int64_t k2w8_shape_gemm_pitch(int64_t k) {
  if (k < 0 || k > kShapeDomain) return -1;
  return (k % 8192 == 0) ? k + 64 : k;
}

// src/kernels/shape.rs:12-16
int64_t k2w8_shape_capacity(int64_t tokens) {
  if (tokens < 0 || tokens > kShapeDomain) return -1;
  int64_t tiles = (tokens + 16 + 31) / 32 * 32;
  int64_t blocks = (tokens + 63) / 64 * 64;
  return tiles > blocks ? tiles : blocks;
}

// src/kernels/shape.rs:110-112
int64_t k2w8_shape_gemm_grid_rows(int64_t tokens) {
  if (tokens < 0 || tokens > kShapeDomain) return -1;
  return (tokens + 255) / 256;
}

// src/kernels/shape.rs:97-99
int k2w8_shape_gemm_schedule_rows(int64_t tokens) { return tokens >= 4096 ? 1 : 0; }

int64_t k2w8_shape_gemm_rows(void) { return 256; }
int64_t k2w8_shape_gemm_m_group(void) { return 4; }
int64_t k2w8_shape_tokens_min(void) { return 16; }
int64_t k2w8_shape_tokens_max(void) { return 16896; }

}  // extern "C"
