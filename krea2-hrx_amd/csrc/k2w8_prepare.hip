// Activation prepares of the W8A8 path for gfx950: form a token's row (modulated
// RMSNorm, plain f16, or attention x sigmoid(gate)), rotate it by the group-256
// regular Hadamard H4 (x) H4 (x) H4 (x) H4, and quantise it per token to int8
// with an f32 scale.
//
// One 256-lane workgroup (four wave64s) per token. The rotation runs on sets of
// sixteen values held in registers, two radix-4 stages per set:
//   pass 1: a lane owns 16 adjacent elements (a "run"): stages of stride 1 and 4;
//   pass 2: a lane owns the 16 elements b, b+16, ..., b+240 of a 256-group: the
//           stages of stride 16 and 64 are again register strides 1 and 4.
// The row crosses LDS (f32) once between the passes and once more before the
// quantiser, which works on runs again so each lane stores 16 contiguous bytes.
//
// Reference arithmetic: kernels/prepare_{norm,plain,gated}_i8.loom (each step
// below cites its lines).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k2w8_numerics.hpp"
#include "k2w8_internal.hpp"

namespace k2w8 {

namespace {

constexpr int kThreads = 256;

enum PrepareKind { kNorm = 0, kPlain = 1, kGated = 2 };

// LDS index of row element e: four floats of padding after every 64 so that
// the sixteen lanes of one 256-group (pass 2) and the next group start 16 banks apart.
__device__ __forceinline__ int lds_index(int e) { return e + ((e >> 6) << 2); }

// One radix-4 stage of H4 on quads (v[i], v[i+s], v[i+2s], v[i+3s]) of a 16-set,
// with the reference's operation order (kernels/prepare_norm_i8.loom:194-201):
//   o0 = (e0+e1)+(e2-e3), o1 = (e0+e1)-(e2-e3), o2 = (e0-e1)+(e2+e3), o3 = (e2+e3)-(e0-e1).
// The plain prepare scales each output by 1/4 and rounds it to f16
// (kernels/prepare_plain_i8.loom:120-127).
template <int S, bool kF16Quarter>
__device__ __forceinline__ void radix4(float (&v)[16]) {
#pragma unroll
  for (int block = 0; block < 16; block += 4 * S) {
#pragma unroll
    for (int c = 0; c < S; ++c) {
      const int i = block + c;
      float e0 = v[i], e1 = v[i + S], e2 = v[i + 2 * S], e3 = v[i + 3 * S];
      float s01 = e0 + e1, s23 = e2 + e3, d01 = e0 - e1, d23 = e2 - e3;
      float o0 = s01 + d23, o1 = s01 - d23, o2 = d01 + s23, o3 = s23 - d01;
      if (kF16Quarter) {
        o0 = f16_round(o0 * 0.25f);
        o1 = f16_round(o1 * 0.25f);
        o2 = f16_round(o2 * 0.25f);
        o3 = f16_round(o3 * 0.25f);
      }
      v[i] = o0;
      v[i + S] = o1;
      v[i + 2 * S] = o2;
      v[i + 3 * S] = o3;
    }
  }
}

__device__ __forceinline__ void unpack_halves(const uint4 &p, uint16_t (&out)[8]) {
  const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = (uint16_t)(w[i] & 0xffffu);
    out[2 * i + 1] = (uint16_t)(w[i] >> 16);
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v = fmaxf(v, __shfl_xor(v, s));
  return v;
}

struct PrepareArgs {
  const uint16_t *h;      // norm: bf16 h; plain: f16 h; gated: f16 attn
  const uint16_t *gate;   // gated only
  const float *norm_scale, *mod_scale, *mod_shift;  // norm only
  int8_t *q;
  float *q_scale;
  int width, out_stride, gate_stride;
  float eps;
};

template <int kKind>
__global__ __launch_bounds__(kThreads) void prepare_kernel(PrepareArgs args) {
  extern __shared__ float row_lds[];
  __shared__ float partial[8];
  const int lane = threadIdx.x;
  const int64_t token = blockIdx.x;
  const int width = args.width;
  const int runs = width >> 4;

  float rms_inv = 0.0f;
  if (kKind == kNorm) {
    // Sum of squares in the reference's lane layout (kernels/prepare_norm_i8.loom:90-101):
    // lane L accumulates eight partials over chunks L, L+256, ... of 8 values.
    const uint16_t *hr = args.h + token * width;
    const int chunks = width >> 3;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c = lane; c < chunks; c += kThreads) {
      uint16_t x[8];
      unpack_halves(*reinterpret_cast<const uint4 *>(hr + c * 8), x);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float xf = bf16_value(x[e]);
        float sq = xf * xf;
        acc[e] = acc[e] + sq;
      }
    }
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = s + acc[e];
    // Each half of a wave64 is one of the reference's 32-lane waves: xor butterfly
    // with strides 1..16 stays inside the half.
#pragma unroll
    for (int stride = 1; stride < 32; stride <<= 1) s = s + __shfl_xor(s, stride);
    if ((lane & 31) == 0) partial[lane >> 5] = s;
    __syncthreads();
    // :132-143, in the reference's explicit order.
    float pair0 = partial[0] + partial[4], pair1 = partial[1] + partial[5];
    float pair2 = partial[2] + partial[6], pair3 = partial[3] + partial[7];
    float total = (pair0 + pair2) + (pair1 + pair3);
    float mean = total / (float)width;
    float mean_eps = mean + args.eps;
    rms_inv = 1.0f / __builtin_sqrtf(mean_eps);
  }

  // Pass 1: form runs of 16 adjacent elements, stages of stride 1 and 4.
  for (int r = lane; r < runs; r += kThreads) {
    const int e0 = r << 4;
    float v[16];
    if (kKind == kNorm) {
      // :145-170
      const uint16_t *hr = args.h + token * width + e0;
      uint16_t x[16];
      unpack_halves(*reinterpret_cast<const uint4 *>(hr), *reinterpret_cast<uint16_t(*)[8]>(x));
      unpack_halves(*reinterpret_cast<const uint4 *>(hr + 8),
                    *reinterpret_cast<uint16_t(*)[8]>(x + 8));
      const float4 *ns4 = reinterpret_cast<const float4 *>(args.norm_scale + e0);
      const float4 *ms4 = reinterpret_cast<const float4 *>(args.mod_scale + e0);
      const float4 *sh4 = reinterpret_cast<const float4 *>(args.mod_shift + e0);
      float ns[16], ms[16], sh[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float4 a = ns4[i], b = ms4[i], c = sh4[i];
        ns[4 * i] = a.x; ns[4 * i + 1] = a.y; ns[4 * i + 2] = a.z; ns[4 * i + 3] = a.w;
        ms[4 * i] = b.x; ms[4 * i + 1] = b.y; ms[4 * i + 2] = b.z; ms[4 * i + 3] = b.w;
        sh[4 * i] = c.x; sh[4 * i + 1] = c.y; sh[4 * i + 2] = c.z; sh[4 * i + 3] = c.w;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float xf = bf16_value(x[i]);
        float n = xf * rms_inv;
        float ns1 = ns[i] + 1.0f;
        float normed = bf16_round(n * ns1);
        float ms1 = bf16_round(ms[i] + 1.0f);
        float scaled = bf16_round(normed * ms1);
        v[i] = bf16_round(scaled + sh[i]);
      }
    } else if (kKind == kPlain) {
      // kernels/prepare_plain_i8.loom:89-90
      const uint16_t *hr = args.h + token * width + e0;
      uint16_t x[16];
      unpack_halves(*reinterpret_cast<const uint4 *>(hr), *reinterpret_cast<uint16_t(*)[8]>(x));
      unpack_halves(*reinterpret_cast<const uint4 *>(hr + 8),
                    *reinterpret_cast<uint16_t(*)[8]>(x + 8));
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = f16_value(x[i]);
    } else {
      // kernels/prepare_gated_i8.loom:86-108
      const uint16_t *ar = args.h + token * width + e0;
      const uint16_t *gr = args.gate + token * (int64_t)args.gate_stride + e0;
      uint16_t a[16], g[16];
      unpack_halves(*reinterpret_cast<const uint4 *>(ar), *reinterpret_cast<uint16_t(*)[8]>(a));
      unpack_halves(*reinterpret_cast<const uint4 *>(ar + 8),
                    *reinterpret_cast<uint16_t(*)[8]>(a + 8));
      unpack_halves(*reinterpret_cast<const uint4 *>(gr), *reinterpret_cast<uint16_t(*)[8]>(g));
      unpack_halves(*reinterpret_cast<const uint4 *>(gr + 8),
                    *reinterpret_cast<uint16_t(*)[8]>(g + 8));
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float af = bf16_round(f16_value(a[i]));
        float sig = bf16_round(sigmoid(f16_value(g[i])));
        v[i] = bf16_round(af * sig);
      }
    }
    radix4<1, kKind == kPlain>(v);
    radix4<4, kKind == kPlain>(v);
#pragma unroll
    for (int i = 0; i < 16; ++i) row_lds[lds_index(e0 + i)] = v[i];
  }
  __syncthreads();

  // Pass 2: sets {b + 16j} of each 256-group, stages of stride 16 and 64.
  float amax = 0.0f;
  for (int s = lane; s < runs; s += kThreads) {
    const int base = ((s >> 4) << 8) + (s & 15);
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = row_lds[lds_index(base + 16 * j)];
    radix4<1, kKind == kPlain>(v);
    radix4<4, kKind == kPlain>(v);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      amax = fmaxf(amax, fabsf(v[j]));
      row_lds[lds_index(base + 16 * j)] = v[j];
    }
  }
  amax = wave_max(amax);
  if ((lane & 63) == 0) partial[lane >> 6] = amax;
  __syncthreads();

  // Scale (kernels/prepare_plain_i8.loom:294-299, kernels/prepare_norm_i8.loom:322-327).
  const float rotation_scale = (kKind == kPlain) ? 16.0f : 0.0625f;
  float row_max = fmaxf(fmaxf(partial[0], partial[1]), fmaxf(partial[2], partial[3]));
  row_max = row_max * rotation_scale;
  float safe = fmaxf(row_max, 1e-30f);
  float scale = safe / 127.0f;
  float inv = rotation_scale / scale;

  // Quantise runs of 16 and store 16 bytes per lane (:301-340, bytes low first).
  int8_t *qr = args.q + token * (int64_t)args.out_stride;
  for (int r = lane; r < runs; r += kThreads) {
    const int e0 = r << 4;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        float x = row_lds[lds_index(e0 + 4 * i + b)];
        float qv = __builtin_rintf(x * inv);
        qv = fmaxf(qv, -127.0f);
        qv = fminf(qv, 127.0f);
        word |= ((uint32_t)(int)qv & 0xffu) << (8 * b);
      }
      w[i] = word;
    }
    *reinterpret_cast<uint4 *>(qr + e0) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (lane == 0) args.q_scale[token] = scale;
}

}  // namespace

hipError_t launch_prepare(int kind, hipStream_t stream, int64_t tokens, const PrepareLaunch &p) {
  PrepareArgs a;
  a.h = static_cast<const uint16_t *>(p.h);
  a.gate = static_cast<const uint16_t *>(p.gate);
  a.norm_scale = p.norm_scale;
  a.mod_scale = p.mod_scale;
  a.mod_shift = p.mod_shift;
  a.q = p.q;
  a.q_scale = p.q_scale;
  a.width = (int)p.width;
  a.out_stride = (int)p.out_stride;
  a.gate_stride = (int)p.gate_stride;
  a.eps = p.eps;
  const size_t lds = (size_t)(p.width + (p.width >> 6) * 4) * sizeof(float);
  dim3 grid((unsigned)tokens), block(kThreads);
  switch (kind) {
    case kNorm:
      hipLaunchKernelGGL(prepare_kernel<kNorm>, grid, block, lds, stream, a);
      break;
    case kPlain:
      hipLaunchKernelGGL(prepare_kernel<kPlain>, grid, block, lds, stream, a);
      break;
    default:
      hipLaunchKernelGGL(prepare_kernel<kGated>, grid, block, lds, stream, a);
      break;
  }
  return hipGetLastError();
}

hipError_t configure_prepare_lds() {
  // The widest row, 32768 f32 values plus four floats of padding per 64.
  const int max_lds = (32768 + (32768 >> 6) * 4) * (int)sizeof(float);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(prepare_kernel<kNorm>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute(reinterpret_cast<const void *>(prepare_kernel<kPlain>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute(reinterpret_cast<const void *>(prepare_kernel<kGated>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
}

}  // namespace k2w8
