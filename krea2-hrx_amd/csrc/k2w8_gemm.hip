// INT8 GEMM family of the W8A8 path for gfx950 (CDNA4):
//   acc[m][n] = sum_k A[m][k] * W[n][k]   (exact int32, v_mfma_i32_32x32x32_i8)
// followed by a fused dequantising epilogue (plain f16, bf16 gated residual in
// place, SwiGLU, or plain + bias).
//
// Workgroup tile BM x BN with a 128-byte K step; both operands are K-contiguous
// rows, staged through LDS in a 16-byte-chunk XOR swizzle and double buffered:
// the next K step's global loads are in flight while the current step's MFMAs
// run. Each wave64 owns a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks.
// Workgroups are numbered XCD-major (consecutive tiles land on one XCD's L2),
// then grouped m_group m-tiles per sweep of n.
//
// Reference: kernels/gemm_i8_256.loom (tile, raster groups :98-132, ghost rows
// :169-216, epilogue :558-629), kernels/gemm_i8_resid_256.loom:607-635,
// kernels/gemm_i8_swiglu_256.loom:569-660.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k2w8_internal.hpp"
#include "k2w8_numerics.hpp"

namespace k2w8 {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBK = 128;  // bytes of K per stage
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

struct GemmArgs {
  const int8_t *a, *w;
  const float *w_scale, *a_scale;
  void *c;
  const float *gate;
  const uint16_t *bias;
  int m, n, k, lda, m_group;
};

// Byte offset of 16-byte chunk `c` (0..7) of staged row `r`: chunks of eight
// consecutive rows are permuted so a column of chunks spans all banks.
__device__ __forceinline__ int swz(int r, int c) { return (r << 7) | (((c ^ r) & 7) << 4); }

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM *WN * 64) void gemm_kernel(GemmArgs g) {
  constexpr int kThreads = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave sub-tile
  constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 blocks per wave
  constexpr int kAChunks = BM * (kBK / 16) / kThreads;
  constexpr int kBChunks = BN * (kBK / 16) / kThreads;
  constexpr int kStage = (BM + BN) * kBK;
  static_assert(kAChunks * kThreads == BM * 8 && kBChunks * kThreads == BN * 8, "chunking");
  extern __shared__ __align__(16) uint8_t smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;

  // Tile of this workgroup.
  const int tiles_m = (g.m + BM - 1) / BM, tiles_n = g.n / BN;
  const int total = tiles_m * tiles_n;
  int bid = blockIdx.x;
  const int per_xcd = total / kXcds;
  if (bid < per_xcd * kXcds) bid = (bid % kXcds) * per_xcd + bid / kXcds;
  const int span = g.m_group * tiles_n;
  const int group = bid / span, in_group = bid - group * span;
  const int first_m = group * g.m_group;
  const int rows_in_group = min(tiles_m - first_m, g.m_group);
  const int tm = first_m + in_group % rows_in_group;
  const int tn = in_group / rows_in_group;
  const int m0 = tm * BM, n0 = tn * BN;

  // Global -> LDS staging: chunk q = tid + i*kThreads is row q/8, 16-byte chunk q%8.
  // Ghost rows past m read row m-1; their results are never stored.
  uint32_t a_off[kAChunks], b_off[kBChunks];
  int a_lds[kAChunks], b_lds[kBChunks];
#pragma unroll
  for (int i = 0; i < kAChunks; ++i) {
    int q = tid + i * kThreads, r = q >> 3, c = q & 7;
    int gr = min(m0 + r, g.m - 1);
    a_off[i] = (uint32_t)gr * (uint32_t)g.lda + (uint32_t)(c * 16);
    a_lds[i] = swz(r, c);
  }
#pragma unroll
  for (int i = 0; i < kBChunks; ++i) {
    int q = tid + i * kThreads, r = q >> 3, c = q & 7;
    b_off[i] = (uint32_t)(n0 + r) * (uint32_t)g.lda + (uint32_t)(c * 16);
    b_lds[i] = BM * kBK + swz(r, c);
  }

  uint4 ra[kAChunks], rb[kBChunks];
  auto load_global = [&](int kt) {
    const uint32_t ko = (uint32_t)kt * kBK;
#pragma unroll
    for (int i = 0; i < kAChunks; ++i)
      ra[i] = *reinterpret_cast<const uint4 *>(g.a + (a_off[i] + ko));
#pragma unroll
    for (int i = 0; i < kBChunks; ++i)
      rb[i] = *reinterpret_cast<const uint4 *>(g.w + (b_off[i] + ko));
  };
  auto store_lds = [&](int stage) {
    uint8_t *base = smem + stage * kStage;
#pragma unroll
    for (int i = 0; i < kAChunks; ++i) *reinterpret_cast<uint4 *>(base + a_lds[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < kBChunks; ++i) *reinterpret_cast<uint4 *>(base + b_lds[i]) = rb[i];
  };

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  const int wm = wave / WN, wn = wave % WN;
  const int fr = lane & 31, kh = lane >> 5;
  const int kt_count = g.k / kBK;

  load_global(0);
  store_lds(0);
  __syncthreads();

  for (int kt = 0; kt < kt_count; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < kt_count) load_global(kt + 1);
    const uint8_t *sa = smem + cur * kStage;
    const uint8_t *sb = sa + BM * kBK;
#pragma unroll
    for (int s = 0; s < kBK / 32; ++s) {
      const int kc = 2 * s + kh;
      v4i af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const v4i *>(sa + swz(wm * WTM + i * 32 + fr, kc));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const v4i *>(sb + swz(wn * WTN + j * 32 + fr, kc));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < kt_count) store_lds(cur ^ 1);
    __syncthreads();
  }

  // Epilogue. Accumulator register e of block (i, j) holds row
  // (e/4)*8 + kh*4 + e%4 and column fr of the block.
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * WTN + j * 32 + fr;
    const float ws = (EPI == kEpiAcc) ? 1.0f : g.w_scale[n];
    float gate_n = 0.0f, bias_n = 0.0f;
    if (EPI == kEpiResid) gate_n = g.gate[n];
    if (EPI == kEpiBias) bias_n = f16_value(g.bias[n]);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * WTM + i * 32 + (e >> 2) * 8 + kh * 4 + (e & 3);
        const bool live = m < g.m;
        const float as = (EPI == kEpiAcc) ? 1.0f : g.a_scale[live ? m : g.m - 1];
        const float prod = (float)acc[i][j][e] * ws;
        if (EPI == kEpiAcc) {
          if (live) static_cast<int32_t *>(g.c)[(int64_t)m * g.n + n] = acc[i][j][e];
        } else if (EPI == kEpiPlain) {
          if (live)
            static_cast<uint16_t *>(g.c)[(int64_t)m * g.n + n] = f16_bits(bf16_round(prod * as));
        } else if (EPI == kEpiBias) {
          if (live)
            static_cast<uint16_t *>(g.c)[(int64_t)m * g.n + n] =
                f16_bits(bf16_round(prod * as + bias_n));
        } else if (EPI == kEpiResid) {
          if (live) {
            uint16_t *x = static_cast<uint16_t *>(g.c) + (int64_t)m * g.n + n;
            float lin = bf16_round(prod * as);
            float gated = bf16_round(lin * gate_n);
            float prior = bf16_value(*x);
            *x = bf16_bits(prior + gated);
          }
        } else {  // SwiGLU: columns fr < 16 are gates, fr >= 16 the matching ups
          const float v = bf16_round(prod * as);
          const float partner = __shfl_xor(v, 16);
          if (live && (fr & 16) == 0) {
            const float sg = v;
            const float silu = bf16_round(sg * sigmoid(sg));
            const float out = bf16_round(silu * partner);
            const int o = ((n0 + wn * WTN + j * 32) >> 1) + (fr & 15);
            static_cast<uint16_t *>(g.c)[(int64_t)m * (g.n >> 1) + o] = f16_bits(out);
          }
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
struct TileConfig {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr size_t kLds = 2 * (size_t)(BM + BN) * kBK;
};

template <int BM, int BN, int WM, int WN>
hipError_t launch_tile(int epi, hipStream_t stream, const GemmArgs &a) {
  using T = TileConfig<BM, BN, WM, WN>;
  const int tiles = ((a.m + BM - 1) / BM) * (a.n / BN);
  dim3 grid(tiles), block(T::kThreads);
  switch (epi) {
    case kEpiPlain:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, kEpiPlain>), grid, block, T::kLds, stream, a);
      break;
    case kEpiResid:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, kEpiResid>), grid, block, T::kLds, stream, a);
      break;
    case kEpiSwiglu:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, kEpiSwiglu>), grid, block, T::kLds, stream, a);
      break;
    case kEpiBias:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, kEpiBias>), grid, block, T::kLds, stream, a);
      break;
    default:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, kEpiAcc>), grid, block, T::kLds, stream, a);
      break;
  }
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN>
hipError_t set_lds_tile() {
  using T = TileConfig<BM, BN, WM, WN>;
  const void *fns[5] = {reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, kEpiPlain>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, kEpiResid>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, kEpiSwiglu>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, kEpiBias>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, kEpiAcc>)};
  for (const void *f : fns) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::kLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t configure_gemm_lds() {
  hipError_t e = set_lds_tile<256, 256, 2, 4>();
  if (e != hipSuccess) return e;
  return set_lds_tile<256, 128, 4, 2>();
}

hipError_t launch_gemm(int epilogue, hipStream_t stream, const GemmLaunch &l) {
  GemmArgs a;
  a.a = l.a;
  a.w = l.w;
  a.w_scale = l.w_scale;
  a.a_scale = l.a_scale;
  a.c = l.c;
  a.gate = l.gate;
  a.bias = static_cast<const uint16_t *>(l.bias);
  a.m = (int)l.m;
  a.n = (int)l.n;
  a.k = (int)l.k;
  a.lda = (int)l.lda;
  a.m_group = l.m_group;
  const int64_t big_tiles = ((l.m + 255) / 256) * (l.n / 256);
  if (l.n % 256 == 0 && big_tiles >= 256) return launch_tile<256, 256, 2, 4>(epilogue, stream, a);
  return launch_tile<256, 128, 4, 2>(epilogue, stream, a);
}

}  // namespace k2w8
