// Building blocks shared by the INT8 GEMM kernels for gfx950: arguments, the LDS
// swizzle of staged K-contiguous rows, the global -> LDS transfers and their waits,
// the XCD-aware tile order and the fragment reads of one 32-byte K slice.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k2w8 {
namespace gemm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin
constexpr int kCusPerXcd = 32;  // MI355X: 256 CUs

struct GemmArgs {
  const int8_t *a, *w;
  const float *w_scale, *a_scale;
  void *c;
  const float *gate;
  const uint16_t *bias;
  int m, n, k, lda, m_group;
  // Row stride of c in output elements (n, or n/2 for SwiGLU, unless the launch covers
  // a column range of a wider output).
  int ldc = 0;
  // Split K: workgroup row blockIdx.y runs K steps [y * k_split_steps, ...) and writes
  // its int32 partial sums (the kEpiAcc output) at c + y * split_stride elements.
  // 0 = no split.
  int k_split_steps = 0;
  int64_t split_stride = 0;
};

// Staged operand rows are BK bytes = BK/16 chunks of 16 bytes. The chunk index is
// XORed with bits of the row so that the consecutive rows one LDS cycle serves (one
// chunk each) land on distinct banks.
template <int BK>
__device__ __forceinline__ int swz_key(int r) {
  return (r >> 1) & (BK / 16 - 1);
}

// A pointer the compiler may hold in VGPRs, as the scalar-register operand the
// transfer instructions need (it is the same for every lane).
__device__ __forceinline__ const void *uniform_ptr(const void *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void *>(((uint64_t)hi << 32) | lo);
}

// One 16-byte-per-lane global -> LDS transfer (global_load_lds_dwordx4): lane l
// writes LDS bytes [lds + 16 l, lds + 16 l + 16) from global address base + voff.
// Issued through asm so that the waits for it are placed by hand (the compiler
// would otherwise wait for every transfer in flight before any LDS read).
__device__ __forceinline__ void dma16(uint32_t lds, const int8_t *base, uint32_t voff) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(lds) : "memory");
}

// The 4-byte form: lane l writes LDS bytes [lds + 4 l, lds + 4 l + 4).
__device__ __forceinline__ void dma4(uint32_t lds, const void *base, uint32_t voff) {
  asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Tile of workgroup `bid`: XCD-major renumbering, then m_group m-tiles per n sweep.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int m_group, int &tm,
                                        int &tn) {
  const int total = tiles_m * tiles_n;
  const int per_xcd = total / kXcds;
  if (bid < per_xcd * kXcds) bid = (bid % kXcds) * per_xcd + bid / kXcds;
  const int span = m_group * tiles_n;
  const int group = bid / span, in_group = bid - group * span;
  const int first_m = group * m_group;
  const int rows_in_group = min(tiles_m - first_m, m_group);
  tm = first_m + in_group % rows_in_group;
  tn = in_group / rows_in_group;
}

// Output tile and K split of workgroup (x, y) of a split-K grid (tiles x splits).
// Workgroups go to the XCDs in turn (linear id mod kXcds); XCD j takes one contiguous
// run of the work order, which is m-tile fastest, then n-tile, then split. The m-tiles
// of one weight slice then share an XCD's L2, and each XCD reads the A columns of one
// or two K splits only (M=256 down projection: 50 -> 32 MB read past the L2s).
__device__ __forceinline__ void split_tile_of(int x, int y, int tiles, int splits, int tiles_m, int &tm,
                                              int &tn, int &split) {
  const int total = tiles * splits, linear = y * tiles + x;
  const int xcd = linear % kXcds, base = total / kXcds, rem = total - base * kXcds;
  const int w = xcd * base + min(xcd, rem) + linear / kXcds;
  tm = w % tiles_m;
  const int rest = w / tiles_m, tiles_n = tiles / tiles_m;
  tn = rest % tiles_n;
  split = rest / tiles_n;
}

// This wave's A and B fragments of one 32-byte K slice: LDS chunk offset `c` of each
// fragment row.
template <int FM, int FN>
__device__ __forceinline__ void read_frags(v4i (&af)[FM], v4i (&bf)[FN], const uint8_t *stage,
                                           const int (&a_row_off)[FM], const int (&b_row_off)[FN],
                                           int c) {
#pragma unroll
  for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const v4i *>(stage + a_row_off[i] + c);
#pragma unroll
  for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const v4i *>(stage + b_row_off[j] + c);
}

}  // namespace gemm
}  // namespace k2w8
