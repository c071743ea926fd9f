// Host-side interface between the C ABI (k2w8_api.cpp) and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
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

enum Epilogue { kEpiPlain = 0, kEpiResid = 1, kEpiSwiglu = 2, kEpiBias = 3, kEpiAcc = 4 };

struct GemmLaunch {
  const int8_t *a = nullptr, *w = nullptr;
  const float *w_scale = nullptr, *a_scale = nullptr;
  void *c = nullptr;
  const float *gate = nullptr;   // resid
  const void *bias = nullptr;    // bias
  int64_t m = 0, n = 0, k = 0, lda = 0;
  int m_group = 4;
};

hipError_t launch_gemm(int epilogue, hipStream_t stream, const GemmLaunch &g);
// Few-token kernel (any m; chosen by launch_gemm for small m).
hipError_t launch_skinny(int epilogue, hipStream_t stream, const GemmLaunch &g);
hipError_t configure_gemm_lds();

// bf16 <-> f16 transport: direction 1 bf16 -> f16, 2 f16 -> bf16.
hipError_t launch_transport(int direction, hipStream_t stream, int64_t count, const void *x,
                            void *out);

// Multiprocessor (CU) count of the current device, cached per device ordinal.
int device_cus();

// The split-K GEMMs' int32 partial-sum workspace of the current device: allocated on
// first use (never while `stream` is capturing; nullptr then, and the GEMM runs
// without split-K), kept until the process ends.
size_t splitk_workspace_bytes();
void *splitk_workspace(hipStream_t stream);

}  // namespace k2w8
