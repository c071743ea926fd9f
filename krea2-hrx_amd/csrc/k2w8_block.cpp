// The W8A8 stages of a transformer block (Session::block, src/session/mod.rs:671-840)
// over caller-owned session buffers, the block loop recorded once into a hipGraph and
// replayed (src/session/mod.rs:596-616), and a per-stage profile of one eager pass
// (src/session/mod.rs:618-647, 449-479).
//
// Host code only: every launch goes through the library's own entry points, so the
// argument checks and kernels are those of the single-kernel calls. The attention step
// between gemm_qkvg and prepare_gated (q/k norm + rope, V transpose, f16 attention)
// runs when the caller provides its workspaces (buffers->q set); otherwise the caller
// runs its own attention between k2w8_block_pre_attention and
// k2w8_block_post_attention, leaving the output in attn_gu.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "krea2_w8a8.h"
#include "k2w8_internal.hpp"

int k2w8_fail_invalid(const char *message);
int k2w8_fail_runtime(const char *stage, hipError_t e);
int k2w8_succeed();
int k2w8_prime_launches(void *stream);

namespace {

constexpr int kModRows = 6;  // prescale, preshift, pregate, postscale, postshift, postgate
// Bounds of a block call's shape: the prepares' token limit and the widest operand any
// of its GEMMs or prepares accepts; and of the block index (a row of the modulation
// table).
constexpr int64_t kMaxBlockTokens = int64_t(1) << 20, kMaxBlockWidth = 65536;
constexpr int64_t kMaxBlockIndex = int64_t(1) << 20;

int check_cfg(const k2w8_block_cfg *c, const char *stage) {
  char msg[256];
  if (!c) {
    snprintf(msg, sizeof msg, "%s: null configuration", stage);
    return k2w8_fail_invalid(msg);
  }
  // Bounded first, so that the arithmetic below cannot overflow; the stage entry
  // points then check each launch's own limits.
  if (c->tokens < 1 || c->tokens > kMaxBlockTokens || c->hidden < 256 || c->hidden > kMaxBlockWidth ||
      c->inter < 256 || c->inter > kMaxBlockWidth || c->qkvg < c->hidden || c->qkvg > kMaxBlockWidth ||
      c->gate_offset < 0 || c->gate_offset > c->qkvg - c->hidden) {
    snprintf(msg, sizeof msg,
             "%s: shape must have tokens in 1..%lld, hidden, inter and qkvg in 256..%lld, and the "
             "gate half (gate_offset + hidden) inside qkvg",
             stage, (long long)kMaxBlockTokens, (long long)kMaxBlockWidth);
    return k2w8_fail_invalid(msg);
  }
  return K2W8_OK;
}

const float *mod_row(const k2w8_block_buffers *b, const k2w8_block_cfg *c, int64_t index, int part) {
  return b->mods + (index * kModRows + part) * c->hidden;
}

// One stage: a label (the reference's stage names) and the call that launches it.
struct Stage {
  const char *label;
  int (*run)(void *stream, const k2w8_block_cfg *c, int64_t index, const k2w8_block_weights *w,
             const k2w8_block_buffers *b);
};

int stage_prepare(void *s, const k2w8_block_cfg *c, int64_t i, const k2w8_block_weights *w,
                  const k2w8_block_buffers *b) {
  const k2w8_prepare_norm_cfg cfg = {c->hidden, k2w8_shape_gemm_pitch(c->hidden), c->eps};
  return k2w8_prepare_norm_i8(s, &cfg, c->tokens, b->x, w->prenorm, mod_row(b, c, i, 0),
                              mod_row(b, c, i, 1), b->a_q, b->a_s);
}

int stage_qkvg(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *w,
               const k2w8_block_buffers *b) {
  const int64_t pitch = k2w8_shape_gemm_pitch(c->hidden);
  const k2w8_gemm_cfg cfg = {c->hidden, c->qkvg, pitch, k2w8_shape_gemm_m_group(), 0};
  return k2w8_gemm_i8(s, &cfg, c->tokens, b->a_q, w->qkvg_q, w->qkvg_s, b->a_s, b->fused);
}

int stage_gated(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *,
                const k2w8_block_buffers *b) {
  const k2w8_prepare_gated_cfg cfg = {c->hidden, k2w8_shape_gemm_pitch(c->hidden), c->qkvg};
  const uint16_t *gate = static_cast<const uint16_t *>(b->fused) + c->gate_offset;
  return k2w8_prepare_gated_i8(s, &cfg, c->tokens, b->attn_gu, gate, b->a_q, b->a_s);
}

int stage_wo(void *s, const k2w8_block_cfg *c, int64_t i, const k2w8_block_weights *w,
             const k2w8_block_buffers *b) {
  const int64_t pitch = k2w8_shape_gemm_pitch(c->hidden);
  const k2w8_gemm_cfg cfg = {c->hidden, c->hidden, pitch, k2w8_shape_gemm_m_group(), 0};
  return k2w8_gemm_i8_resid(s, &cfg, c->tokens, b->a_q, w->wo_q, w->wo_s, b->a_s, b->x,
                            mod_row(b, c, i, 2));
}

int stage_post(void *s, const k2w8_block_cfg *c, int64_t i, const k2w8_block_weights *w,
               const k2w8_block_buffers *b) {
  const k2w8_prepare_norm_cfg cfg = {c->hidden, k2w8_shape_gemm_pitch(c->hidden), c->eps};
  return k2w8_prepare_norm_i8(s, &cfg, c->tokens, b->x, w->postnorm, mod_row(b, c, i, 3),
                              mod_row(b, c, i, 4), b->a_q, b->a_s);
}

int stage_gu(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *w,
             const k2w8_block_buffers *b) {
  const int64_t pitch = k2w8_shape_gemm_pitch(c->hidden);
  const k2w8_gemm_cfg cfg = {c->hidden, 2 * c->inter, pitch, k2w8_shape_gemm_m_group(), 0};
  return k2w8_gemm_i8_swiglu(s, &cfg, c->tokens, b->a_q, w->gu_q, w->gu_s, b->a_s, b->attn_gu);
}

int stage_swiglu(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *,
                 const k2w8_block_buffers *b) {
  const k2w8_prepare_plain_cfg cfg = {c->inter, k2w8_shape_gemm_pitch(c->inter)};
  return k2w8_prepare_plain_i8(s, &cfg, c->tokens, b->attn_gu, b->a_q, b->a_s);
}

int stage_down(void *s, const k2w8_block_cfg *c, int64_t i, const k2w8_block_weights *w,
               const k2w8_block_buffers *b) {
  const int64_t pitch = k2w8_shape_gemm_pitch(c->inter);
  const k2w8_gemm_cfg cfg = {c->inter, c->hidden, pitch, k2w8_shape_gemm_m_group(),
                             k2w8_shape_gemm_schedule_rows(c->tokens)};
  return k2w8_gemm_i8_resid_256x256(s, &cfg, c->tokens, b->a_q, w->down_q, w->down_s, b->a_s,
                                    b->x, mod_row(b, c, i, 5));
}

// The attention step (src/session/mod.rs:713-755). Heads: q_heads = hidden/128 at
// column 0 of `fused`, kv_heads = (gate_offset - hidden)/256 of k at column hidden and
// of v after them.
struct Heads {
  int64_t q, kv, group, capacity;
};

Heads heads_of(const k2w8_block_cfg *c) {
  Heads h;
  h.q = c->hidden / 128;
  h.kv = (c->gate_offset - c->hidden) / 256;
  h.group = h.kv > 0 ? h.q / h.kv : 0;
  h.capacity = k2w8_shape_capacity(c->tokens);
  return h;
}

int stage_rope(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *w,
               const k2w8_block_buffers *b) {
  const Heads h = heads_of(c);
  const k2w8_rope_qknorm_cfg cfg = {c->qkvg, h.q, h.kv, c->hidden, c->eps};
  return k2w8_rope_qknorm_f16(s, &cfg, c->tokens, b->fused, w->qnorm, w->knorm, b->cos, b->sin,
                              b->q, b->k, b->v);
}

int stage_vt(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *,
             const k2w8_block_buffers *b) {
  const Heads h = heads_of(c);
  const k2w8_v_transpose_cfg cfg = {h.kv * 128, h.capacity};
  return k2w8_v_transpose(s, &cfg, c->tokens, b->v, b->vt);
}

int stage_attention(void *s, const k2w8_block_cfg *c, int64_t, const k2w8_block_weights *,
                    const k2w8_block_buffers *b) {
  const Heads h = heads_of(c);
  // kernels/blocks.rs:94-103: q_stride = out_stride = hidden, kv_stride = kv width.
  const k2w8_attention_cfg cfg = {c->hidden, h.kv * 128, c->hidden, c->tokens, h.capacity,
                                  0.08838834764831845f};
  return k2w8_attention_f16_grouped(s, &cfg, c->tokens, h.kv, h.group, b->q, b->k, b->vt,
                                    b->attn_gu);
}

const Stage kPre[] = {{"prepare", stage_prepare}, {"gemm qkvg", stage_qkvg}};
const Stage kAttn[] = {{"qk norm + rope", stage_rope},
                       {"V transpose", stage_vt},
                       {"f16 attention", stage_attention}};
const Stage kPost[] = {{"prepare gated", stage_gated},
                       {"gemm wo + residual", stage_wo},
                       {"prepare", stage_post},
                       {"gemm gate|up + swiglu", stage_gu},
                       {"prepare swiglu", stage_swiglu},
                       {"gemm down + residual", stage_down}};

template <size_t N>
int run_stages(const Stage (&stages)[N], void *stream, const k2w8_block_cfg *c, int64_t index,
               const k2w8_block_weights *w, const k2w8_block_buffers *b) {
  for (const Stage &st : stages) {
    const int rc = st.run(stream, c, index, w, b);
    if (rc != K2W8_OK) return rc;
  }
  return K2W8_OK;
}

int check_call(const k2w8_block_cfg *c, int64_t index, const k2w8_block_weights *w,
               const k2w8_block_buffers *b, const char *stage) {
  int rc = check_cfg(c, stage);
  if (rc != K2W8_OK) return rc;
  char msg[256];
  if (!w || !b || !b->mods) {
    snprintf(msg, sizeof msg, "%s: null weights, buffers or modulation table", stage);
    return k2w8_fail_invalid(msg);
  }
  if (index < 0 || index >= kMaxBlockIndex) {
    snprintf(msg, sizeof msg, "%s: block index must be in 0..%lld, got %lld", stage,
             (long long)(kMaxBlockIndex - 1), (long long)index);
    return k2w8_fail_invalid(msg);
  }
  return K2W8_OK;
}

bool with_attention(const k2w8_block_buffers *b) { return b && b->q; }

int check_attention(const k2w8_block_cfg *c, const k2w8_block_weights *w,
                    const k2w8_block_buffers *b, const char *stage) {
  char msg[256];
  const Heads h = heads_of(c);
  if (c->hidden % 128 || (c->gate_offset - c->hidden) % 256 || h.kv < 1 ||
      (h.group != 1 && h.group != 2 && h.group != 4) || h.group * h.kv != h.q) {
    snprintf(msg, sizeof msg,
             "%s: attention needs hidden/128 query heads and (gate_offset - hidden)/256 "
             "key-value heads in a ratio of 1, 2 or 4",
             stage);
    return k2w8_fail_invalid(msg);
  }
  if (c->tokens < 16) {
    snprintf(msg, sizeof msg, "%s: attention needs tokens >= 16", stage);
    return k2w8_fail_invalid(msg);
  }
  if (!w->qnorm || !w->knorm || !b->q || !b->k || !b->v || !b->vt || !b->cos || !b->sin) {
    snprintf(msg, sizeof msg, "%s: null qnorm/knorm or attention workspace", stage);
    return k2w8_fail_invalid(msg);
  }
  return K2W8_OK;
}

int check_block(const k2w8_block_cfg *c, int64_t index, const k2w8_block_weights *w,
                const k2w8_block_buffers *b, const char *stage) {
  int rc = check_call(c, index, w, b, stage);
  if (rc == K2W8_OK && with_attention(b)) rc = check_attention(c, w, b, stage);
  return rc;
}

// One block: pre-attention stages, the attention step when its workspaces are given,
// post-attention stages.
int run_block(void *stream, const k2w8_block_cfg *c, int64_t index, const k2w8_block_weights *w,
              const k2w8_block_buffers *b) {
  int rc = run_stages(kPre, stream, c, index, w, b);
  if (rc == K2W8_OK && with_attention(b)) rc = run_stages(kAttn, stream, c, index, w, b);
  if (rc == K2W8_OK) rc = run_stages(kPost, stream, c, index, w, b);
  return rc;
}

constexpr int64_t kPreCount = sizeof kPre / sizeof kPre[0];
constexpr int64_t kAttnCount = sizeof kAttn / sizeof kAttn[0];
constexpr int64_t kPostCount = sizeof kPost / sizeof kPost[0];
constexpr int64_t kStageCount = kPreCount + kAttnCount + kPostCount;

const Stage &stage_at(int64_t k) {
  if (k < kPreCount) return kPre[k];
  if (k < kPreCount + kAttnCount) return kAttn[k - kPreCount];
  return kPost[k - kPreCount - kAttnCount];
}

}  // namespace

struct k2w8_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  // The split-K workspace the recorded GEMMs write: the graph's own, so a replay on
  // any stream never shares partial sums with eager calls on the recording stream.
  void *workspace = nullptr;
  ~k2w8_graph() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (workspace) (void)hipFree(workspace);
  }
};

extern "C" {

int k2w8_block_pre_attention(void *stream, const k2w8_block_cfg *cfg, int64_t index,
                             const k2w8_block_weights *weights, const k2w8_block_buffers *buffers) {
  int rc = check_call(cfg, index, weights, buffers, "block_pre_attention");
  if (rc != K2W8_OK) return rc;
  return run_stages(kPre, stream, cfg, index, weights, buffers);
}

int k2w8_block_attention(void *stream, const k2w8_block_cfg *cfg, int64_t index,
                         const k2w8_block_weights *weights, const k2w8_block_buffers *buffers) {
  const char *stage = "block_attention";
  int rc = check_call(cfg, index, weights, buffers, stage);
  if (rc != K2W8_OK) return rc;
  if (!with_attention(buffers)) return k2w8_fail_invalid("block_attention: null q workspace");
  if ((rc = check_attention(cfg, weights, buffers, stage)) != K2W8_OK) return rc;
  return run_stages(kAttn, stream, cfg, index, weights, buffers);
}

int k2w8_block_post_attention(void *stream, const k2w8_block_cfg *cfg, int64_t index,
                              const k2w8_block_weights *weights, const k2w8_block_buffers *buffers) {
  int rc = check_call(cfg, index, weights, buffers, "block_post_attention");
  if (rc != K2W8_OK) return rc;
  return run_stages(kPost, stream, cfg, index, weights, buffers);
}

int k2w8_blocks_record(void *stream, const k2w8_block_cfg *cfg, int64_t layers,
                       const k2w8_block_weights *weights, const k2w8_block_buffers *buffers,
                       k2w8_graph **out) {
  const char *stage = "blocks_record";
  if (!out) return k2w8_fail_invalid("blocks_record: null output");
  *out = nullptr;
  if (layers < 1 || layers > kMaxBlockIndex) return k2w8_fail_invalid("blocks_record: layers must be in 1..2^20");
  for (int64_t i = 0; i < layers; ++i) {
    int rc = check_block(cfg, i, weights + i, buffers, stage);
    if (rc != K2W8_OK) return rc;
  }
  if (!stream)
    return k2w8_fail_invalid("blocks_record: recording needs a created stream (not the null stream)");
  // One-time set-up (kernel attributes, device queries) must not happen inside capture.
  int rc = k2w8_prime_launches(stream);
  if (rc != K2W8_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto g = std::make_unique<k2w8_graph>();
  const size_t ws_bytes = k2w8::splitk_workspace_bytes();
  hipError_t e = hipMalloc(&g->workspace, ws_bytes);
  if (e != hipSuccess) return k2w8_fail_runtime("blocks_record: the graph's split-K workspace", e);
  e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
  k2w8::splitk_install(k2w8::Workspace{g->workspace, ws_bytes});
  for (int64_t i = 0; i < layers && rc == K2W8_OK; ++i) rc = run_block(stream, cfg, i, weights + i, buffers);
  k2w8::splitk_install(k2w8::Workspace{});
  e = hipStreamEndCapture(s, &g->graph);
  if (rc != K2W8_OK) return rc;
  if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
  *out = g.release();
  return k2w8_succeed();
}

int k2w8_graph_launch(void *stream, k2w8_graph *graph) {
  if (!graph || !graph->exec) return k2w8_fail_invalid("graph_launch: null graph");
  hipError_t e = hipGraphLaunch(graph->exec, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return k2w8_fail_runtime("graph_launch", e);
  return k2w8_succeed();
}

void k2w8_graph_free(k2w8_graph *graph) { delete graph; }

int k2w8_blocks_profile(void *stream, const k2w8_block_cfg *cfg, int64_t layers,
                        const k2w8_block_weights *weights, const k2w8_block_buffers *buffers,
                        double *stage_us, int64_t stage_count) {
  const char *stage = "blocks_profile";
  if (!stage_us || stage_count < kStageCount)
    return k2w8_fail_invalid("blocks_profile: stage_us must hold k2w8_block_stage_count() values");
  if (layers < 1 || layers > kMaxBlockIndex) return k2w8_fail_invalid("blocks_profile: layers must be in 1..2^20");
  for (int64_t i = 0; i < layers; ++i) {
    int rc = check_block(cfg, i, weights + i, buffers, stage);
    if (rc != K2W8_OK) return rc;
  }
  const bool attention = with_attention(buffers);
  std::vector<int64_t> order;  // the stages this pass runs, in order
  for (int64_t k = 0; k < kStageCount; ++k) {
    const bool is_attn = k >= kPreCount && k < kPreCount + kAttnCount;
    stage_us[k] = is_attn && !attention ? -1.0 : 0.0;
    if (!is_attn || attention) order.push_back(k);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::vector<hipEvent_t> ev(order.size() * (size_t)layers + 1, nullptr);
  for (auto &x : ev) {
    const hipError_t e = hipEventCreate(&x);
    if (e != hipSuccess) {
      for (auto &y : ev)
        if (y) (void)hipEventDestroy(y);
      return k2w8_fail_runtime(stage, e);
    }
  }
  int rc = K2W8_OK;
  size_t at = 0;
  hipError_t e = hipEventRecord(ev[at++], s);
  for (int64_t i = 0; i < layers && rc == K2W8_OK && e == hipSuccess; ++i)
    for (int64_t k : order) {
      if ((rc = stage_at(k).run(stream, cfg, i, weights + i, buffers)) != K2W8_OK) break;
      if ((e = hipEventRecord(ev[at++], s)) != hipSuccess) break;
    }
  if (rc == K2W8_OK && e == hipSuccess) e = hipEventSynchronize(ev[at - 1]);
  if (rc == K2W8_OK && e == hipSuccess) {
    for (size_t k = 1; k < at; ++k) {
      float ms = 0.0f;
      if ((e = hipEventElapsedTime(&ms, ev[k - 1], ev[k])) != hipSuccess) break;
      stage_us[order[(k - 1) % order.size()]] += 1e3 * (double)ms;
    }
  }
  for (auto &x : ev) (void)hipEventDestroy(x);
  if (rc != K2W8_OK) return rc;
  if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
  return k2w8_succeed();
}

int64_t k2w8_block_stage_count(void) { return kStageCount; }

const char *k2w8_block_stage_label(int64_t index) {
  if (index < 0 || index >= kStageCount) return nullptr;
  return stage_at(index).label;
}

}  // extern "C"
