// The C ABI's argument validation (krea2-hrx_amd/csrc/k2w8_api.cpp) against what the
// kernel launchers assume, built with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_abi_sanitized.py. The launchers are replaced by stubs that check their
// preconditions: the shape limits, strides, 32-bit offset bounds, token ranges, pointer
// presence and alignment each kernel relies on. The driver makes 400000 calls of the
// GEMM, prepare and one-call linear entry points, and 100000 of the block entry points
// (k2w8_block.cpp, which chain them with the attention step's), with edge values,
// random values and mostly-valid configurations with one field off; every call the
// ABI accepts must meet the preconditions, and none may trip a sanitizer.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <algorithm>
#include <random>
#include "krea2_w8a8.h"
#include "k2w8_internal.hpp"

static long g_gemm = 0, g_prep = 0, g_other = 0, g_bad = 0;
#define REQ(c) do { if (!(c)) { fprintf(stderr, "violated: %s (line %d)\n", #c, __LINE__); ++g_bad; } } while (0)
static bool al(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// No GPU here: the entry points' per-device set-up sees device 0 (this definition
// takes the place of the HIP runtime's for the code linked into this program).
extern "C" hipError_t hipGetDevice(int *device) {
  *device = 0;
  return hipSuccess;
}

namespace k2w8 {
hipError_t configure_gemm_lds() { return hipSuccess; }
hipError_t configure_prepare_lds() { return hipSuccess; }
hipError_t configure_fused_lds() { return hipSuccess; }
int device_cus() { return 256; }
hipError_t prepare_gated_ready(hipStream_t) { return hipSuccess; }
hipError_t launch_gemm(int epi, hipStream_t, const GemmLaunch &l) {
  ++g_gemm;
  REQ(epi >= 0 && epi <= kEpiAcc);
  REQ(l.m >= 1 && l.m <= (1 << 24));
  REQ(l.n >= 128 && l.n <= 32768 && l.n % 128 == 0);
  REQ(l.k >= 128 && l.k <= 65536 && l.k % 128 == 0);
  REQ(l.lda >= l.k && l.lda <= 65536 && l.lda % 64 == 0);
  REQ(l.m * l.lda < (1ll << 31) && l.n * l.lda < (1ll << 31) && l.m * l.n < (1ll << 31));
  REQ(l.m_group >= 1 && l.m_group <= 4);
  REQ(l.a && l.w && l.w_scale && l.a_scale && l.c);
  REQ(al(l.a, 16) && al(l.w, 16) && al(l.w_scale, 16) && al(l.c, 16) && al(l.a_scale, 4));
  if (epi == kEpiResid) REQ(l.gate && al(l.gate, 16));
  if (epi == kEpiBias) REQ(l.bias && al(l.bias, 16));
  return hipSuccess;
}
hipError_t launch_prepare(int kind, hipStream_t, int64_t tokens, const PrepareLaunch &p) {
  ++g_prep;
  REQ(kind >= 0 && kind <= 2);
  REQ(tokens >= 1 && tokens <= (1 << 20));
  REQ(p.width >= 256 && p.width <= 32768 && p.width % 256 == 0);
  REQ(p.out_stride >= p.width && p.out_stride <= 65536 && p.out_stride % 64 == 0);
  REQ(p.h && p.q && p.q_scale && al(p.h, 16) && al(p.q, 16) && al(p.q_scale, 4));
  if (kind == 0) REQ(p.norm_scale && p.mod_scale && p.mod_shift && p.eps >= 0.0f);
  if (kind == 2) REQ(p.gate && al(p.gate, 16) && p.gate_stride >= p.width && p.gate_stride % 8 == 0);
  return hipSuccess;
}
hipError_t launch_prepare_gemm(int, hipStream_t, int64_t, const PrepareLaunch &, const GemmLaunch &) {
  return hipErrorNotSupported;
}
hipError_t launch_probe_mfma(hipStream_t, int64_t, int64_t, int, uint32_t, int32_t *) { return hipSuccess; }
hipError_t launch_rope_qknorm(hipStream_t, const RopeLaunch &l) {
  ++g_other;
  REQ(l.tokens >= 1 && l.tokens <= (1 << 20));
  REQ(l.q_heads >= 1 && l.kv_heads >= 1 && (l.q_heads + 2 * l.kv_heads) * l.tokens < (1ll << 32));
  REQ(l.row_stride % 8 == 0 && l.q_heads * 128 <= l.row_stride && l.k_offset % 8 == 0 &&
      l.k_offset + 2 * l.kv_heads * 128 <= l.row_stride);
  REQ(l.qkv && l.q_scale && l.k_scale && l.cos && l.sin && l.q_out && l.k_out && l.v_out);
  REQ(al(l.qkv, 16) && al(l.q_out, 16) && al(l.k_out, 16) && al(l.v_out, 16) && al(l.cos, 16) && al(l.sin, 16));
  return hipSuccess;
}
hipError_t launch_sigmoid(hipStream_t, int64_t, const float *, float *) { return hipSuccess; }
hipError_t launch_transport(int, hipStream_t, int64_t, const void *, void *) { return hipSuccess; }
hipError_t launch_v_transpose(hipStream_t, int64_t rows, int64_t width, int64_t capacity, const void *x,
                              void *out) {
  ++g_other;
  REQ(rows >= 1 && rows <= capacity && capacity % 8 == 0 && width % 8 == 0 && width >= 8);
  REQ(width * capacity < (1ll << 40) && x && out && al(x, 16) && al(out, 16));
  return hipSuccess;
}
hipError_t launch_attention(hipStream_t, const AttentionLaunch &l) {
  ++g_other;
  REQ(l.group == 1 || l.group == 2 || l.group == 4);
  REQ(l.tokens >= 16 && l.capacity >= l.tokens + 16 && l.capacity % 16 == 0 && l.capacity <= (1 << 20));
  REQ(l.rows_out >= 1 && l.rows_out <= l.tokens);
  REQ(l.q_stride % 128 == 0 && l.kv_stride % 128 == 0 && l.out_stride % 128 == 0);
  REQ(l.kv_heads >= 1 && l.kv_heads * 128 <= l.kv_stride && l.group * l.kv_heads * 128 <= l.q_stride &&
      l.group * l.kv_heads * 128 <= l.out_stride);
  REQ(l.scale > 0.0f && l.q && l.k && l.vt && l.out && al(l.q, 16) && al(l.k, 16) && al(l.vt, 16) &&
      al(l.out, 16));
  return hipSuccess;
}
hipError_t splitk_register(hipStream_t, void *, size_t) { return hipSuccess; }
size_t splitk_workspace_bytes() { return 64u << 20; }
Workspace splitk_static_scratch(hipError_t *e) { *e = hipSuccess; return Workspace{(void *)0x100000, 16u << 20}; }
hipError_t splitk_static_ordered(hipStream_t, const std::function<hipError_t()> &launch) { return launch(); }
void splitk_install(Workspace) {}
bool gemm_streams(int, const GemmLaunch &l, int64_t) { return l.m <= 32; }
}  // namespace k2w8

int main() {
  std::mt19937_64 rng(99);
  const int64_t edge[] = {-1, 0, 1, 63, 64, 127, 128, 192, 255, 256, 2048, 2560, 3072, 4096, 8192, 8256,
                          9728, 12288, 16384, 16448, 32768, 32896, 65472, 65536, 65600, 1 << 20, (1 << 20) + 1,
                          1 << 24, (1 << 24) + 1, 1ll << 31, 1ll << 40, INT64_MAX, INT64_MIN};
  auto pick = [&]() -> int64_t { return rng() % 4 ? edge[rng() % (sizeof edge / 8)] : (int64_t)(rng() % 70000) - 100; };
  auto ptr = [&]() -> void * {
    switch (rng() % 8) { case 0: return nullptr; case 1: return (void *)0x10004; case 2: return (void *)0x10002; default: return (void *)0x10000; }
  };
  const float epss[] = {1e-6f, 0.0f, -1.0f, __builtin_nanf(""), __builtin_inff()};
  for (int it = 0; it < 400000; ++it) {
    k2w8_gemm_cfg g{pick(), pick(), pick(), pick() % 6, pick() % 3};
    int64_t m = pick();
    if (rng() % 10 < 7) {  // mostly valid: the accept side of every bound
      g.k_size = 128 * (1 + (int64_t)(rng() % 512));
      g.n_size = 128 * (1 + (int64_t)(rng() % 256));
      g.k_stride = std::min<int64_t>(65536, g.k_size + 64 * (int64_t)(rng() % 3));
      g.m_group = 1 + (int64_t)(rng() % 4);
      g.schedule_rows = (int64_t)(rng() % 2);
      m = 1 + (int64_t)(rng() % (rng() % 2 ? 5000 : (1 << 24)));
      switch (rng() % 6) {  // then one field off by a little
        case 0: g.k_size += (rng() % 2 ? 64 : -128); break;
        case 1: g.k_stride -= 64; break;
        case 2: m = rng() % 2 ? 0 : m; break;
        default: break;
      }
    }
    switch (rng() % 9) {
      case 0: k2w8_gemm_i8(nullptr, &g, m, (int8_t *)ptr(), (int8_t *)ptr(), (float *)ptr(), (float *)ptr(), ptr()); break;
      case 1: k2w8_gemm_i8_resid(nullptr, &g, m, (int8_t *)ptr(), (int8_t *)ptr(), (float *)ptr(), (float *)ptr(), ptr(), (float *)ptr()); break;
      case 2: k2w8_gemm_i8_swiglu(nullptr, &g, m, (int8_t *)ptr(), (int8_t *)ptr(), (float *)ptr(), (float *)ptr(), ptr()); break;
      case 3: k2w8_gemm_i8_bias(nullptr, &g, m, (int8_t *)ptr(), (int8_t *)ptr(), (float *)ptr(), (float *)ptr(), ptr(), ptr()); break;
      case 4: k2w8_gemm_i8_noalloc(nullptr, &g, m, (int8_t *)ptr(), (int8_t *)ptr(), (float *)ptr(), (float *)ptr(), ptr()); break;
      case 5: {
        k2w8_prepare_norm_cfg c{pick(), pick(), epss[rng() % 5]};
        if (rng() % 2) { c.width = g.k_size - g.k_size % 256; c.out_stride = g.k_stride; }
        k2w8_prepare_norm_i8(nullptr, &c, m, ptr(), (float *)ptr(), (float *)ptr(), (float *)ptr(), (int8_t *)ptr(), (float *)ptr());
        k2w8_linear_norm_swiglu_i8(nullptr, &c, &g, m, ptr(), (float *)ptr(), (float *)ptr(), (float *)ptr(), (int8_t *)ptr(),
                                   (float *)ptr(), (int8_t *)ptr(), (float *)ptr(), ptr());
        break;
      }
      case 6: {
        k2w8_prepare_plain_cfg c{pick(), pick()};
        if (rng() % 2) { c.width = g.k_size - g.k_size % 256; c.out_stride = g.k_stride; }
        k2w8_prepare_plain_i8(nullptr, &c, m, ptr(), (int8_t *)ptr(), (float *)ptr());
        k2w8_linear_plain_resid_i8(nullptr, &c, &g, m, ptr(), (int8_t *)ptr(), (float *)ptr(), (int8_t *)ptr(), (float *)ptr(),
                                   ptr(), (float *)ptr());
        break;
      }
      case 7: {
        k2w8_prepare_gated_cfg c{pick(), pick(), pick()};
        if (rng() % 2) { c.width = g.k_size - g.k_size % 256; c.out_stride = g.k_stride; c.gate_stride = c.width + 8 * (int64_t)(rng() % 3); }
        k2w8_prepare_gated_i8(nullptr, &c, m, ptr(), ptr(), (int8_t *)ptr(), (float *)ptr());
        k2w8_linear_gated_resid_i8(nullptr, &c, &g, m, ptr(), ptr(), (int8_t *)ptr(), (float *)ptr(), (int8_t *)ptr(),
                                   (float *)ptr(), ptr(), (float *)ptr());
        break;
      }
      default: {
        k2w8_prepare_norm_cfg c{pick(), pick(), epss[rng() % 5]};
        k2w8_linear_norm_i8(nullptr, &c, &g, m, ptr(), (float *)ptr(), (float *)ptr(), (float *)ptr(), (int8_t *)ptr(),
                            (float *)ptr(), (int8_t *)ptr(), (float *)ptr(), ptr());
      }
    }
  }
  // The kernel choice (k2w8_gemm_choose): plan_tiles and the split rule on any
  // accepted shape, CU count and workspace size.
  long chosen = 0;
  for (int it = 0; it < 200000; ++it) {
    k2w8_gemm_cfg g{128 * (1 + (int64_t)(rng() % 512)), 128 * (1 + (int64_t)(rng() % 256)), 0, 4, 0};
    g.k_stride = g.k_size;
    if (rng() % 8 == 0) g.k_size = pick();
    const int64_t m = rng() % 8 ? 1 + (int64_t)(rng() % (1 << 24)) : pick();
    const int64_t cus = rng() % 8 ? 1 + (int64_t)(rng() % 4096) : pick();
    const int64_t ws = rng() % 8 ? (int64_t)(rng() % (1ll << 36)) : pick();
    k2w8_gemm_choice out;
    const int32_t required = (int32_t)(rng() % 2);
    if (k2w8_gemm_choose((int32_t)(rng() % 6) - 1 + 1, m, &g, cus, ws, required, &out) == K2W8_OK) {
      ++chosen;
      REQ(out.kernel >= (required ? -1 : 0) && out.kernel <= 3);
      if (out.kernel == -1) REQ(2 * m * g.n_size * 4 > ws);
      if (out.kernel > 0) REQ(out.tile_m >= 64 && out.tile_n >= 64 && out.stages >= 2);
      if (out.kernel == 2) REQ(out.n_big > 0 && out.n_big < g.n_size && out.n_big % 256 == 0);
      if (out.kernel == 3) REQ(out.splits >= 2 && out.split_steps >= 1 && (int64_t)out.splits * out.split_steps * 128 >= g.k_size &&
                               2 * m * g.n_size * 4 <= ws);
    }
  }
  printf("choices %ld, ", chosen);

  // The block entry points (k2w8_block.cpp), which chain the stage calls above and
  // the attention step's, over edge, huge and mostly-valid block shapes and indices.
  const int64_t bedge[] = {-1, 0, 1, 15, 16, 128, 255, 256, 384, 512, 1024, 3072, 6144, 9216, 12288, 15360,
                           16384, 1 << 20, 1ll << 31, 1ll << 40, INT64_MAX - 5, INT64_MAX, INT64_MIN};
  auto bpick = [&]() -> int64_t { return bedge[rng() % (sizeof bedge / 8)]; };
  long blocks_accepted = 0;
  for (int it = 0; it < 100000; ++it) {
    k2w8_block_cfg c{bpick(), bpick(), bpick(), bpick(), bpick(), 1e-5f};
    if (rng() % 2) {
      c.tokens = 1 + (int64_t)(rng() % 5000);
      c.hidden = 256 * (1 + (int64_t)(rng() % 24));
      c.inter = 256 * (1 + (int64_t)(rng() % 64));
      c.gate_offset = c.hidden + 256 * (int64_t)(rng() % 8);
      c.qkvg = c.gate_offset + c.hidden + (int64_t)(rng() % 3) * 128;
    }
    k2w8_block_weights w;
    memset(&w, 0, sizeof w);
    const void **wp = reinterpret_cast<const void **>(&w);
    for (size_t i = 0; i < sizeof w / sizeof(void *); ++i) wp[i] = rng() % 10 ? (void *)0x10000 : nullptr;
    k2w8_block_buffers b;
    memset(&b, 0, sizeof b);
    void **bp = reinterpret_cast<void **>(&b);
    for (size_t i = 0; i < sizeof b / sizeof(void *); ++i) bp[i] = rng() % 10 ? (void *)0x10000 : nullptr;
    const int64_t index = rng() % 4 ? (int64_t)(rng() % 64) : bpick();
    int rc;
    switch (rng() % 3) {
      case 0: rc = k2w8_block_pre_attention(nullptr, &c, index, &w, &b); break;
      case 1: rc = k2w8_block_attention(nullptr, &c, index, &w, &b); break;
      default: rc = k2w8_block_post_attention(nullptr, &c, index, &w, &b); break;
    }
    blocks_accepted += rc == K2W8_OK;
  }
  // The shape rules outside their domain.
  for (int64_t v : bedge) {
    (void)k2w8_shape_gemm_pitch(v);
    (void)k2w8_shape_capacity(v);
    (void)k2w8_shape_gemm_grid_rows(v);
    (void)k2w8_shape_gemm_schedule_rows(v);
  }
  printf("gemm launches %ld, prepare launches %ld, other launches %ld, blocks accepted %ld, violations %ld\n",
         g_gemm, g_prep, g_other, blocks_accepted, g_bad);
  return g_bad ? 1 : 0;
}
