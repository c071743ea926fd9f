// bf16 <-> f16 transport of the W8A8 projection's caller (the reference's
// krea2_lora_transport, kernels/native/lora_transport.loom:15-41): every element is
// widened exactly to f32 and rounded to the other 16-bit format, round to nearest even.
//   direction 1: bf16 -> f16 (values past 65504 become infinities)
//   direction 2: f16 -> bf16
//
// HBM-bound elementwise pass: each lane moves 8 elements (16-byte loads and stores),
// with a scalar tail for counts that are not a multiple of 8. Grid-stride, so any count
// runs with a bounded grid.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k2w8_internal.hpp"
#include "k2w8_numerics.hpp"

namespace k2w8 {

namespace {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

template <int kDirection>
__device__ __forceinline__ uint32_t convert2(uint32_t w) {
  if (kDirection == 1) {
    const float a = __uint_as_float(w << 16), b = __uint_as_float(w & 0xffff0000u);
    return f16_pack2(a, b);
  }
  const float a = f16_value((uint16_t)(w & 0xffffu)), b = f16_value((uint16_t)(w >> 16));
  return bf16_pack2(a, b);
}

template <int kDirection>
__device__ __forceinline__ uint16_t convert1(uint16_t x) {
  if (kDirection == 1) return f16_bits(bf16_value(x));
  return (uint16_t)(bf16_pack2(f16_value(x), 0.0f) & 0xffffu);
}

template <int kDirection>
__global__ __launch_bounds__(256) void transport_kernel(const uint16_t *x, uint16_t *out,
                                                        int64_t count) {
  const int64_t vecs = count >> 3;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < vecs; v += step) {
    const v4u in = reinterpret_cast<const v4u *>(x)[v];
    v4u o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = convert2<kDirection>(in[i]);
    reinterpret_cast<v4u *>(out)[v] = o;
  }
  // Tail: the last count % 8 elements, by the first threads of block 0.
  const int64_t tail = vecs << 3;
  if (blockIdx.x == 0 && tail + threadIdx.x < count)
    out[tail + threadIdx.x] = convert1<kDirection>(x[tail + threadIdx.x]);
}

__global__ __launch_bounds__(256) void sigmoid_kernel(const float *x, float *out, int64_t count) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += step)
    out[i] = sigmoid(x[i]);
}

}  // namespace

// The device sigmoid of the gated prepare and the SwiGLU epilogue, elementwise: lets
// its bits be compared with the CPU definition over any set of inputs.
hipError_t launch_sigmoid(hipStream_t stream, int64_t count, const float *x, float *out) {
  int64_t blocks = (count + 255) / 256;
  const int64_t cap = (int64_t)device_cus() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(sigmoid_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, out, count);
  return hipGetLastError();
}

hipError_t launch_transport(int direction, hipStream_t stream, int64_t count, const void *x,
                            void *out) {
  const int64_t vecs = count >> 3;
  int64_t blocks = (vecs + 255) / 256;
  const int64_t cap = (int64_t)device_cus() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  dim3 grid((unsigned)blocks), block(256);
  const uint16_t *src = static_cast<const uint16_t *>(x);
  uint16_t *dst = static_cast<uint16_t *>(out);
  if (direction == 1)
    hipLaunchKernelGGL(transport_kernel<1>, grid, block, 0, stream, src, dst, count);
  else
    hipLaunchKernelGGL(transport_kernel<2>, grid, block, 0, stream, src, dst, count);
  return hipGetLastError();
}

}  // namespace k2w8
