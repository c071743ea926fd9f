// Split-K for the GEMM family at shapes with too few output tiles to fill the chip
// (the mid-M text-encoder shapes). The tile kernel runs once per K slice and writes
// each slice's exact int32 partial sums to a workspace; this kernel adds the slices
// (integer addition: any order gives the same sums) and applies the epilogue, with
// the same f32 operation sequence as the tile kernels' epilogues
// (kernels/gemm_i8_256.loom:606-626, kernels/gemm_i8_resid_256.loom:623-635,
// kernels/gemm_i8_swiglu_256.loom:640-660).
//
// The workspace of a call is, in order: the buffer a graph recording installs for its
// capture (each recorded graph owns one, so replays never share partial sums with
// eager calls), a buffer the caller registered for (device, stream), or one device
// allocation per (device, stream) made on first use outside any stream capture and
// kept for the life of the process. Calls on one stream are ordered, so they may share
// a stream's workspace; calls on different streams get their own and never race on it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <utility>

#include "k2w8_gemm_common.hpp"
#include "k2w8_internal.hpp"
#include "k2w8_numerics.hpp"

namespace k2w8 {

namespace splitk {

typedef int v4i __attribute__((ext_vector_type(4)));

struct ReduceArgs {
  const int32_t *parts;
  int splits;
  int64_t stride;  // elements between slices
  int m, n;
  const float *w_scale, *a_scale;
  void *c;
  const float *gate;
  const uint16_t *bias;
};

// The slices' loads go out in groups of eight before any of them is waited for: a loop
// of one load and one add per slice waits a full memory round trip per slice (six
// slices: 2.9 us per workgroup).
__device__ __forceinline__ v4i sum_slices(const ReduceArgs &r, int64_t at) {
  v4i acc = {0, 0, 0, 0};
  for (int s0 = 0; s0 < r.splits; s0 += 8) {
    v4i v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = s0 + i < r.splits ? *reinterpret_cast<const v4i *>(r.parts + (s0 + i) * r.stride + at)
                               : v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += v[i];
  }
  return acc;
}

// One work item: four consecutive channels of one row (SwiGLU: four gate channels and
// their four up channels, 16 rows further on in the 32-row group).
template <int EPI>
__global__ __launch_bounds__(256) void reduce_kernel(ReduceArgs r) {
  const int64_t per_row = EPI == kEpiSwiglu ? r.n / 8 : r.n / 4;
  const int64_t total = (int64_t)r.m * per_row;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(t / per_row);
    const int g = (int)(t - (int64_t)m * per_row);
    if (EPI == kEpiSwiglu) {
      const int nb = (g >> 2) * 32 + (g & 3) * 4;  // gate channels nb..nb+3
      const int64_t row = (int64_t)m * r.n;
      const v4i ag = sum_slices(r, row + nb), au = sum_slices(r, row + nb + 16);
      const float as = r.a_scale[m];
      const float4 gs = *reinterpret_cast<const float4 *>(r.w_scale + nb);
      const float4 us = *reinterpret_cast<const float4 *>(r.w_scale + nb + 16);
      const float gsv[4] = {gs.x, gs.y, gs.z, gs.w}, usv[4] = {us.x, us.y, us.z, us.w};
      float gv[4], uv[4];
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        float g0 = ((float)ag[e] * gsv[e]) * as, g1 = ((float)ag[e + 1] * gsv[e + 1]) * as;
        float u0 = ((float)au[e] * usv[e]) * as, u1 = ((float)au[e + 1] * usv[e + 1]) * as;
        bf16_round2(g0, g1);
        bf16_round2(u0, u1);
        gv[e] = g0; gv[e + 1] = g1; uv[e] = u0; uv[e + 1] = u1;
      }
      swiglu_products(gv, uv);
      const uint32_t packed[2] = {f16_pack2(gv[0], gv[1]), f16_pack2(gv[2], gv[3])};
      const int o = (g >> 2) * 16 + (g & 3) * 4;
      *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(r.c) + (int64_t)m * (r.n >> 1) + o) =
          make_uint2(packed[0], packed[1]);
      continue;
    }
    const int nb = g * 4;
    const int64_t at = (int64_t)m * r.n + nb;
    const v4i acc = sum_slices(r, at);
    if (EPI == kEpiAcc) {
      *reinterpret_cast<v4i *>(static_cast<int32_t *>(r.c) + at) = acc;
      continue;
    }
    const float as = r.a_scale[m];
    const float4 w4 = *reinterpret_cast<const float4 *>(r.w_scale + nb);
    const float ws[4] = {w4.x, w4.y, w4.z, w4.w};
    float extra[4] = {0.f, 0.f, 0.f, 0.f};
    if (EPI == kEpiResid) {
      const float4 v = *reinterpret_cast<const float4 *>(r.gate + nb);
      extra[0] = v.x; extra[1] = v.y; extra[2] = v.z; extra[3] = v.w;
    }
    if (EPI == kEpiBias) {
      const uint2 v = *reinterpret_cast<const uint2 *>(r.bias + nb);
      extra[0] = f16_value(v.x & 0xffffu); extra[1] = f16_value(v.x >> 16);
      extra[2] = f16_value(v.y & 0xffffu); extra[3] = f16_value(v.y >> 16);
    }
    uint16_t *out = static_cast<uint16_t *>(r.c) + at;
    uint32_t prior[2] = {0u, 0u};
    if (EPI == kEpiResid) {
      const uint2 p = *reinterpret_cast<const uint2 *>(out);
      prior[0] = p.x;
      prior[1] = p.y;
    }
    uint32_t packed[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      float v0 = ((float)acc[e] * ws[e]) * as, v1 = ((float)acc[e + 1] * ws[e + 1]) * as;
      if (EPI == kEpiBias) {
        v0 = v0 + extra[e];
        v1 = v1 + extra[e + 1];
      }
      bf16_round2(v0, v1);
      if (EPI == kEpiResid) {  // x = bf16(x + bf16(gate * bf16(v)))
        float g0 = v0 * extra[e], g1 = v1 * extra[e + 1];
        bf16_round2(g0, g1);
        const uint32_t w = prior[e >> 1];
        packed[e >> 1] = bf16_pack2(__uint_as_float(w << 16) + g0, __uint_as_float(w & 0xffff0000u) + g1);
      } else {
        packed[e >> 1] = f16_pack2(v0, v1);
      }
    }
    *reinterpret_cast<uint2 *>(out) = make_uint2(packed[0], packed[1]);
  }
}

constexpr size_t kWorkspaceBytes = size_t(64) << 20;
std::mutex g_lock;
// (device, stream) -> the library's own buffer, and -> the caller's registered one
std::map<std::pair<int, uintptr_t>, void *> g_owned;
std::map<std::pair<int, uintptr_t>, Workspace> g_registered;
thread_local Workspace t_installed;

}  // namespace splitk

// Scratch of k2w8_gemm_i8_noalloc: a file-scope device array, so that entry point never
// allocates. 16 MiB holds at least two K slices of every shape the split-K rule picks
// (it splits only when 128x128 tiles cover at most half of the 256 CUs: m x n <= 2^21
// outputs, 8 MiB of int32 per slice). Every call on a device shares that device's copy;
// eager calls are ordered on the device (splitk_static_ordered), captured ones by their
// graph. Each slice overwrites its whole part, so nothing needs clearing between calls.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) int32_t scratch[kScratchBytes / sizeof(int32_t)];

namespace splitk {
struct Scratch {
  void *ptr = nullptr;         // the address of that device's `scratch`
  hipEvent_t last = nullptr;   // the end of the last eager call that used it
};
std::map<int, Scratch> g_scratch;  // device -> its scratch
std::mutex g_order;                // held across one call's wait, launches and record
}  // namespace splitk

Workspace splitk_static_scratch(hipError_t *err) {
  *err = hipSuccess;
  int dev = 0;
  if ((*err = hipGetDevice(&dev)) != hipSuccess) return Workspace{};
  std::lock_guard<std::mutex> guard(splitk::g_lock);
  const auto it = splitk::g_scratch.find(dev);
  if (it != splitk::g_scratch.end()) return Workspace{it->second.ptr, kScratchBytes};
  // The array's name is a host-side stand-in; the device copy's address comes from the
  // runtime, once per device, with that device current. The ordering event is made in
  // the same set-up step.
  splitk::Scratch sc;
  if ((*err = hipGetSymbolAddress(&sc.ptr, HIP_SYMBOL(scratch))) != hipSuccess) return Workspace{};
  if ((*err = hipEventCreateWithFlags(&sc.last, hipEventDisableTiming)) != hipSuccess) return Workspace{};
  splitk::g_scratch[dev] = sc;
  return Workspace{sc.ptr, kScratchBytes};
}

hipError_t splitk_static_ordered(hipStream_t stream, const std::function<hipError_t()> &launch) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipEvent_t last = nullptr;
  {
    std::lock_guard<std::mutex> guard(splitk::g_lock);
    const auto it = splitk::g_scratch.find(dev);
    if (it != splitk::g_scratch.end()) last = it->second.last;
  }
  // (the null stream, torch's default one, is never capturing)
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (stream && (e = hipStreamIsCapturing(stream, &capture)) != hipSuccess) return e;
  if (!last || capture != hipStreamCaptureStatusNone) return launch();
  std::lock_guard<std::mutex> order(splitk::g_order);
  if ((e = hipStreamWaitEvent(stream, last, 0)) != hipSuccess) return e;
  if ((e = launch()) != hipSuccess) return e;
  return hipEventRecord(last, stream);
}

size_t splitk_workspace_bytes() { return splitk::kWorkspaceBytes; }

void splitk_install(Workspace ws) { splitk::t_installed = ws; }

hipError_t splitk_register(hipStream_t stream, void *ptr, size_t bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const auto key = std::make_pair(dev, reinterpret_cast<uintptr_t>(stream));
  std::lock_guard<std::mutex> guard(splitk::g_lock);
  if (ptr)
    splitk::g_registered[key] = Workspace{ptr, bytes};
  else
    splitk::g_registered.erase(key);
  return hipSuccess;
}

Workspace splitk_workspace(hipStream_t stream) {
  if (splitk::t_installed.ptr) return splitk::t_installed;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return Workspace{};
  const auto key = std::make_pair(dev, reinterpret_cast<uintptr_t>(stream));
  std::lock_guard<std::mutex> guard(splitk::g_lock);
  const auto reg = splitk::g_registered.find(key);
  if (reg != splitk::g_registered.end()) return reg->second;
  const auto it = splitk::g_owned.find(key);
  if (it != splitk::g_owned.end()) return Workspace{it->second, splitk::kWorkspaceBytes};
  // Never allocate inside a stream capture: the caller then runs without split-K.
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (stream && hipStreamIsCapturing(stream, &status) != hipSuccess) return Workspace{};
  if (status != hipStreamCaptureStatusNone) return Workspace{};
  void *p = nullptr;
  if (hipMalloc(&p, splitk::kWorkspaceBytes) != hipSuccess) {
    (void)hipGetLastError();
    return Workspace{};
  }
  splitk::g_owned[key] = p;
  return Workspace{p, splitk::kWorkspaceBytes};
}

hipError_t launch_splitk_reduce(int epilogue, hipStream_t stream, const int32_t *parts, int splits,
                                int64_t stride, const gemm::GemmArgs &g) {
  splitk::ReduceArgs r;
  r.parts = parts;
  r.splits = splits;
  r.stride = stride;
  r.m = g.m;
  r.n = g.n;
  r.w_scale = g.w_scale;
  r.a_scale = g.a_scale;
  r.c = g.c;
  r.gate = g.gate;
  r.bias = g.bias;
  const int64_t items = (int64_t)g.m * (epilogue == kEpiSwiglu ? g.n / 8 : g.n / 4);
  int64_t blocks = (items + 255) / 256;
  const int64_t cap = (int64_t)device_cus() * 8;
  if (blocks > cap) blocks = cap;
  dim3 grid((unsigned)(blocks > 0 ? blocks : 1)), block(256);
  switch (epilogue) {
    case kEpiPlain: hipLaunchKernelGGL(splitk::reduce_kernel<kEpiPlain>, grid, block, 0, stream, r); break;
    case kEpiResid: hipLaunchKernelGGL(splitk::reduce_kernel<kEpiResid>, grid, block, 0, stream, r); break;
    case kEpiSwiglu: hipLaunchKernelGGL(splitk::reduce_kernel<kEpiSwiglu>, grid, block, 0, stream, r); break;
    case kEpiBias: hipLaunchKernelGGL(splitk::reduce_kernel<kEpiBias>, grid, block, 0, stream, r); break;
    default: hipLaunchKernelGGL(splitk::reduce_kernel<kEpiAcc>, grid, block, 0, stream, r); break;
  }
  return hipGetLastError();
}

}  // namespace k2w8
