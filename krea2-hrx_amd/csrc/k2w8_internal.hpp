// Host-side interface between the C ABI (k2w8_api.cpp) and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <stdint.h>

namespace k2w8 {

struct PrepareLaunch {
  const void *h = nullptr;
  const void *gate = nullptr;
  const float *norm_scale = nullptr, *mod_scale = nullptr, *mod_shift = nullptr;
  int8_t *q = nullptr;
  float *q_scale = nullptr;
  int64_t width = 0, out_stride = 0, gate_stride = 0;
  float eps = 0.0f;
};

// kind: 0 norm, 1 plain, 2 gated
hipError_t launch_prepare(int kind, hipStream_t stream, int64_t tokens, const PrepareLaunch &p);
hipError_t configure_prepare_lds();
// One-time set-up of the gated prepare on the current device (its sigmoid table); not
// inside a stream capture.
hipError_t prepare_gated_ready(hipStream_t stream);

// Device memory for the split-K GEMMs' int32 partial sums.
struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};

enum Epilogue { kEpiPlain = 0, kEpiResid = 1, kEpiSwiglu = 2, kEpiBias = 3, kEpiAcc = 4 };

struct GemmLaunch {
  const int8_t *a = nullptr, *w = nullptr;
  const float *w_scale = nullptr, *a_scale = nullptr;
  void *c = nullptr;
  const float *gate = nullptr;   // resid
  const void *bias = nullptr;    // bias
  int64_t m = 0, n = 0, k = 0, lda = 0;
  int m_group = 4;
  // Split-K workspace for this call; unset (nullptr): splitk_workspace(stream).
  const Workspace *workspace = nullptr;
  // With `workspace`: a shape that would split K into slices that do not fit (fewer
  // than two) fails with hipErrorInvalidValue before any launch, instead of running
  // unsplit.
  bool workspace_required = false;
};

hipError_t launch_gemm(int epilogue, hipStream_t stream, const GemmLaunch &g);
// prepare_norm_i8 (kind 0) or prepare_plain_i8 (kind 1) and gemm_i8 in one persistent
// launch (the wide-tile shapes whose tiles fill whole rounds, prepare width <= 3072);
// hipErrorNotSupported otherwise, having launched nothing.
hipError_t launch_prepare_gemm(int kind, hipStream_t stream, int64_t tokens, const PrepareLaunch &p,
                               const GemmLaunch &g);
// Few-token kernel (any m; chosen by launch_gemm for small m).
bool skinny_streams(int epilogue, const GemmLaunch &g, int64_t cus);
// The few-token kernel's choice (M <= 32, or skinny_streams) with `cus` CUs.
bool gemm_streams(int epilogue, const GemmLaunch &g, int64_t cus);
hipError_t launch_skinny(int epilogue, hipStream_t stream, const GemmLaunch &g);
hipError_t configure_gemm_lds();
// The one-launch prepare -> GEMM kernels' LDS limit, on the current device.
hipError_t configure_fused_lds();
hipError_t configure_skinny_lds();

// bf16 <-> f16 transport: direction 1 bf16 -> f16, 2 f16 -> bf16.
hipError_t launch_sigmoid(hipStream_t stream, int64_t count, const float *x, float *out);
hipError_t launch_probe_mfma(hipStream_t stream, int64_t blocks, int64_t iters, int random, uint32_t seed,
                             int32_t *out);
hipError_t launch_transport(int direction, hipStream_t stream, int64_t count, const void *x,
                            void *out);

// The attention step (rope_qknorm, V transpose, fp16 GQA attention).
struct RopeLaunch {
  const void *qkv = nullptr;
  const float *q_scale = nullptr, *k_scale = nullptr, *cos = nullptr, *sin = nullptr;
  void *q_out = nullptr, *k_out = nullptr, *v_out = nullptr;
  int64_t tokens = 0, row_stride = 0, q_heads = 0, kv_heads = 0, k_offset = 0;
  float eps = 0.0f;
};
hipError_t launch_rope_qknorm(hipStream_t stream, const RopeLaunch &l);
hipError_t launch_v_transpose(hipStream_t stream, int64_t rows, int64_t width, int64_t capacity,
                              const void *x, void *out);
struct AttentionLaunch {
  const void *q = nullptr, *k = nullptr, *vt = nullptr;
  void *out = nullptr;
  int64_t tokens = 0, rows_out = 0, capacity = 0, q_stride = 0, kv_stride = 0, out_stride = 0, kv_heads = 0;
  int64_t group = 4;  // query heads per key-value head: 1, 2 or 4
  float scale = 0.0f;
};
hipError_t launch_attention(hipStream_t stream, const AttentionLaunch &l);

// Multiprocessor (CU) count of the current device, cached per device ordinal.
int device_cus();

// Bytes of the workspace the library allocates for a stream (and for a recorded graph).
size_t splitk_workspace_bytes();
// The workspace of a call on `stream` (current device), in order: the one a recording
// on this thread has installed, the caller's registered for (device, stream), the
// library's own for (device, stream), allocated on first use. Never allocates while
// `stream` is capturing: {nullptr, 0} then, and the GEMM runs without split-K.
Workspace splitk_workspace(hipStream_t stream);
// Register caller-owned memory as the workspace of (current device, stream); a null
// ptr removes the registration.
hipError_t splitk_register(hipStream_t stream, void *ptr, size_t bytes);
// The workspace every split-K call on this thread uses while a recording is being
// captured (nullptr ptr: none installed).
void splitk_install(Workspace ws);
// The allocation-free GEMM entry point's scratch: a static device array, one per
// device. Its address on the current device is looked up once per device; `err`
// receives the lookup's failure.
Workspace splitk_static_scratch(hipError_t *err);
// Orders the eager calls that use the current device's static scratch: `stream` waits
// (on the device, not the host) for the previous such call's work, `launch` enqueues
// this call's, and its end becomes the next call's wait. Inside a stream capture it
// only runs `launch`: the graph orders its own calls, and replays of graphs that use
// the scratch must not overlap one another.
hipError_t splitk_static_ordered(hipStream_t stream, const std::function<hipError_t()> &launch);

}  // namespace k2w8
