// Fused prepare -> GEMM: one persistent launch that first prepares every token row
// (norm or plain prepare into the caller's q / q_scale), meets at a grid-wide barrier,
// then runs the GEMM's output tiles with the plain epilogue. The same device code as
// the separate kernels (prepare_rows, gemm_tile) does the work, so the results are
// bit-identical to k2w8_prepare_*_i8 followed by k2w8_gemm_i8.
//
// The grid is one workgroup of eight waves per CU (the GEMM tile's LDS allows one), so
// every workgroup is resident and the barrier cannot wait on one that never started.
// Workgroup b prepares rows as eight one-wave teams (teams b*8 .. b*8+7 of the
// persistent prepare's order) and then takes tiles b, b + grid, ... of the GEMM's tile
// order. Writes of phase 1 reach the other XCDs through an agent-scope release before
// the barrier; each workgroup acquires after it, before its first tile reads q.
//
// Reference: the prepare -> gemm pair of Session::block / Quantized::forward
// (src/session/mod.rs:671-711, src/training/quantized.rs:66-105), launched as two
// kernels there.
#define K2W8_GEMM_NO_ENTRY
#define K2W8_PREPARE_NO_ENTRY
#include "k2w8_prepare.hip"
#include "k2w8_gemm.hip"

namespace k2w8 {

namespace fused {

// Arrival and departure counts of the grid barrier. Both are zero between launches: the
// last workgroup to depart resets them, so graph replays start from zero too.
__device__ unsigned int g_barrier[2];

// Bound on the barrier's polls (each about a microsecond with the sleep): far past any
// prepare phase, only there so that a broken residency assumption cannot hang the GPU.
constexpr int kBarrierPolls = 1 << 22;

__device__ __forceinline__ void grid_barrier(unsigned int blocks) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(&g_barrier[0], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = 0; i < kBarrierPolls; ++i) {
      if (__hip_atomic_load(&g_barrier[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) >= blocks) break;
      __builtin_amdgcn_s_sleep(8);
    }
    const unsigned int left =
        __hip_atomic_fetch_add(&g_barrier[1], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (left == blocks - 1) {
      __hip_atomic_store(&g_barrier[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&g_barrier[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
}

template <int kKind, int T, int BM, int BN>
__global__ __launch_bounds__(512) void prepare_gemm_kernel(PrepareArgs p, gemm::GemmArgs g,
                                                           int tiles) {
  extern __shared__ __align__(16) uint8_t smem[];
  prepare_rows<kKind, T, true>(p, blockIdx.x, gridDim.x, reinterpret_cast<float4 *>(smem));
  grid_barrier(gridDim.x);
  for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
    gemm::gemm_tile<BM, BN, 4, 2, 128, 2, kEpiPlain>(g, t, smem);
    __syncthreads();  // the next tile's transfers overwrite the epilogue's LDS regions
  }
}

template <int kKind, int T, int BM, int BN>
hipError_t launch(hipStream_t stream, const PrepareArgs &p, const gemm::GemmArgs &g, int cus) {
  const void *fn = reinterpret_cast<const void *>(prepare_gemm_kernel<kKind, T, BM, BN>);
  const size_t stage_lds = (size_t)2 * (BM + BN) * 128 + gemm::EpiOperands<BM, BN>::kBytes +
                           gemm::EpiStaging<BM, BN, 4, 2, 128, 2, 1>::kOverflow;
  const size_t factor_lds = kKind == kNorm ? (size_t)(p.width / 16) * kFactorStride * 16 : 0;
  const size_t lds = stage_lds > factor_lds ? stage_lds : factor_lds;
  static hipError_t configured = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (configured != hipSuccess) return configured;
  const int tiles = ((g.m + BM - 1) / BM) * (g.n / BN);
  hipLaunchKernelGGL((prepare_gemm_kernel<kKind, T, BM, BN>), dim3(cus), dim3(512), lds, stream, p, g,
                     tiles);
  return hipGetLastError();
}

}  // namespace fused

// The fused launch for the wide-tile shapes, with the tile choice of launch_gemm (256x256
// or 256x192 tiles in whole rounds); hipErrorNotSupported for every other shape, which
// the caller then runs as two launches.
hipError_t launch_prepare_gemm(int kind, hipStream_t stream, int64_t tokens,
                               const PrepareLaunch &pl, const GemmLaunch &gl) {
  const int cus = device_cus();
  if (pl.width > 3072 || gl.m != tokens || gl.n % 256 != 0 || gl.lda != pl.out_stride)
    return hipErrorNotSupported;
  const int64_t tm = (gl.m + 255) / 256;
  const int64_t t256 = tm * (gl.n / 256), t192 = gl.n % 192 == 0 ? tm * (gl.n / 192) : 0;
  int bn = 0;
  if (t192 > 0 && t192 % cus == 0 && (t256 % cus != 0 || t192 / cus * 192 < t256 / cus * 256))
    bn = 192;
  else if (t256 % cus == 0)
    bn = 256;
  if (bn == 0) return hipErrorNotSupported;
  PrepareArgs p;
  p.h = static_cast<const uint16_t *>(pl.h);
  p.gate = nullptr;
  p.norm_scale = pl.norm_scale;
  p.mod_scale = pl.mod_scale;
  p.mod_shift = pl.mod_shift;
  p.q = pl.q;
  p.q_scale = pl.q_scale;
  p.tokens = (int)tokens;
  p.width = (int)pl.width;
  p.out_stride = (int)pl.out_stride;
  p.gate_stride = 0;
  p.eps = pl.eps;
  p.wpt = 1;
  p.teams = 8;
  p.one = 1.0f;
  const gemm::GemmArgs g = gemm::args_of(gl, kEpiPlain);
  const int t = (int)((pl.width / 16 + 63) / 64);  // runs of 16 per lane
  if (kind == kNorm) {
    if (t <= 2) return bn == 256 ? fused::launch<kNorm, 2, 256, 256>(stream, p, g, cus)
                                 : fused::launch<kNorm, 2, 256, 192>(stream, p, g, cus);
    return bn == 256 ? fused::launch<kNorm, 3, 256, 256>(stream, p, g, cus)
                     : fused::launch<kNorm, 3, 256, 192>(stream, p, g, cus);
  }
  if (t <= 2) return bn == 256 ? fused::launch<kPlain, 2, 256, 256>(stream, p, g, cus)
                               : fused::launch<kPlain, 2, 256, 192>(stream, p, g, cus);
  return bn == 256 ? fused::launch<kPlain, 3, 256, 256>(stream, p, g, cus)
                   : fused::launch<kPlain, 3, 256, 192>(stream, p, g, cus);
}

}  // namespace k2w8
