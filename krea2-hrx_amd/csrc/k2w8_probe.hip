// The INT8 MFMA rate with nothing else running: back-to-back v_mfma_i32_32x32x32_i8 on
// operands held in registers, no memory traffic in the loop. It measures the ceiling
// the tile GEMM is compared against under the chip's power limit: the MFMA's power
// depends on its operand bits (all-ones bytes against pseudo-random ones), and the
// clock the chip holds follows. Not part of the W8A8 path.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k2w8_internal.hpp"

namespace k2w8 {

namespace probe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Eight independent accumulator chains per wave (two waves per SIMD keep the MFMA pipe
// busy), operands from a per-lane xorshift stream or bytes of 1. Each lane writes the
// sum of its accumulators, so the loop cannot be removed.
constexpr int kChains = 8;

__global__ __launch_bounds__(256) void mfma_i8_kernel(uint32_t seed, int random, int iters, int32_t *out) {
  uint32_t x = (seed ^ ((blockIdx.x * 256u + threadIdx.x) * 0x9E3779B9u)) | 1u;
  auto next = [&] {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return (int)x;
  };
  v4i a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = random ? v4i{next(), next(), next(), next()} : v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
    b[i] = random ? v4i{next(), next(), next(), next()} : v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
  }
  v16i acc[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kChains; ++j)
      acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j & 3], b[j >> 2], acc[j], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace probe

hipError_t launch_probe_mfma(hipStream_t stream, int64_t blocks, int64_t iters, int random, uint32_t seed,
                             int32_t *out) {
  hipLaunchKernelGGL(probe::mfma_i8_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, seed, random,
                     (int)iters, out);
  return hipGetLastError();
}

}  // namespace k2w8
