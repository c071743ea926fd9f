// Fused prepare -> GEMM: one persistent launch that first prepares every token row
// (norm or plain prepare into the caller's q / q_scale), meets at a grid-wide barrier,
// then runs the GEMM's output tiles with the plain epilogue. The same device code as
// the separate kernels (prepare_rows, gemm_tile) does the work, so the results are
// bit-identical to k2w8_prepare_*_i8 followed by k2w8_gemm_i8.
//
// The grid is one workgroup of eight waves per CU (the GEMM tile's LDS allows one).
// Workgroup b prepares rows as eight one-wave teams (teams b*8 .. b*8+7 of the
// persistent prepare's order) and then takes tiles b, b + grid, ... of the GEMM's tile
// order. Writes of phase 1 reach the other XCDs through an agent-scope release before
// the barrier; each workgroup acquires after it, before its first tile reads q.
//
// The barrier waits a bounded time. Its count lives in the launch's own state (the
// stream's workspace, cleared by a one-wave kernel launched just before), so launches
// on other streams never add to it. Every workgroup is resident unless other work
// holds CUs for longer than the bound (another persistent launch on another stream,
// say); a workgroup that gives up then prepares the rows of each of its tiles itself
// before the tile, so its output is still exact, only later.
//
// Reference: the prepare -> gemm pair of Session::block / Quantized::forward
// (src/session/mod.rs:671-711, src/training/quantized.rs:66-105), launched as two
// kernels there.
#define K2W8_GEMM_NO_ENTRY
#define K2W8_PREPARE_NO_ENTRY
#include "k2w8_prepare.hip"
#include "k2w8_gemm.hip"

#include <stdlib.h>

namespace k2w8 {

namespace fused {

// Bound on the barrier's polls by default (each about a microsecond with the sleep):
// far past any prepare phase (tens of microseconds), only there so that a broken
// residency assumption cannot hold the GPU. K2W8_FUSED_BARRIER_POLLS overrides it.
constexpr int kBarrierPolls = 1 << 14;

// Bytes of a launch's barrier state at the start of the stream's workspace: the
// arrival count, cleared by reset_kernel before each launch.
constexpr size_t kStateBytes = 256;

__global__ __launch_bounds__(64) void reset_kernel(unsigned int *state) {
  state[threadIdx.x] = 0u;  // kStateBytes / 4 words
}

// The workgroups meet after the prepare phase. Returns whether every workgroup arrived
// within `polls` polls (the same answer for every thread of the workgroup).
__device__ __forceinline__ bool grid_barrier(unsigned int *arrivals, unsigned int blocks, int polls) {
  __shared__ int passed;
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    int ok = 0;
    for (int i = 0; i < polls; ++i) {
      if (__hip_atomic_load(arrivals, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) >= blocks) {
        ok = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
    passed = ok;
  }
  __syncthreads();
  return passed != 0;
}

// A workgroup whose wait gave up cannot know which rows are prepared, so before each
// of its tiles it prepares the tile's own rows again (the same code, hence the same
// bytes as their producer writes, whenever that runs) and makes them visible to its
// own transfers. The result is that of a passed barrier, only slower.
template <int kKind, int T, int BM>
__device__ __forceinline__ void prepare_tile_rows(const PrepareArgs &p, int tile_m, uint8_t *smem) {
  const int r0 = tile_m * BM;
  PrepareArgs own = p;
  own.h = p.h + (int64_t)r0 * p.width;
  own.q = p.q + (int64_t)r0 * p.out_stride;
  own.q_scale = p.q_scale + r0;
  own.tokens = min(BM, p.tokens - r0);
  prepare_rows<kKind, T, true>(own, 0, 1, reinterpret_cast<float4 *>(smem));
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "agent");
  __syncthreads();  // the prepare's LDS is the tile's staging memory
}

template <int kKind, int T, int BM, int BN>
__global__ __launch_bounds__(512) void prepare_gemm_kernel(PrepareArgs p, gemm::GemmArgs g, int tiles,
                                                           unsigned int *state, int polls) {
  extern __shared__ __align__(16) uint8_t smem[];
  prepare_rows<kKind, T, true>(p, blockIdx.x, gridDim.x, reinterpret_cast<float4 *>(smem));
  const bool passed = grid_barrier(state, gridDim.x, polls);
  const int tiles_m = (g.m + BM - 1) / BM;
  for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
    if (!passed) {
      int tm, tn;
      gemm::tile_of(t, tiles_m, g.n / BN, g.m_group, tm, tn);
      prepare_tile_rows<kKind, T, BM>(p, tm, smem);
    }
    gemm::gemm_tile<BM, BN, 4, 2, 128, 2, kEpiPlain>(g, t, smem);
    __syncthreads();  // the next tile's transfers overwrite the epilogue's LDS regions
  }
}

// Dynamic LDS of the launch: the tile's stages and epilogue, or the norm factors.
template <int kKind, int BM, int BN>
size_t lds_bytes(int width) {
  const size_t stage_lds = (size_t)2 * (BM + BN) * 128 + gemm::EpiOperands<BM, BN>::kBytes +
                           gemm::EpiStaging<BM, BN, 4, 2, 128, 2, 1>::kOverflow;
  const size_t factor_lds = kKind == kNorm ? (size_t)(width / 16) * kFactorStride * 16 : 0;
  return stage_lds > factor_lds ? stage_lds : factor_lds;
}

// The kernels' LDS limit (every launch's need is at most the widest row's, K = 3072).
hipError_t configure() {
  const struct {
    const void *fn;
    size_t lds;
  } kernels[] = {
      {reinterpret_cast<const void *>(prepare_gemm_kernel<kNorm, 2, 256, 192>), lds_bytes<kNorm, 256, 192>(3072)},
      {reinterpret_cast<const void *>(prepare_gemm_kernel<kNorm, 3, 256, 192>), lds_bytes<kNorm, 256, 192>(3072)},
      {reinterpret_cast<const void *>(prepare_gemm_kernel<kPlain, 2, 256, 192>), lds_bytes<kPlain, 256, 192>(3072)},
      {reinterpret_cast<const void *>(prepare_gemm_kernel<kPlain, 3, 256, 192>), lds_bytes<kPlain, 256, 192>(3072)},
  };
  for (const auto &k : kernels) {
    const hipError_t e = hipFuncSetAttribute(k.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)k.lds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int barrier_polls() {
  const char *v = getenv("K2W8_FUSED_BARRIER_POLLS");
  if (!v || !*v) return kBarrierPolls;
  const long n = strtol(v, nullptr, 10);
  return n < 0 ? 0 : (n > (1 << 24) ? (1 << 24) : (int)n);
}

template <int kKind, int T, int BM, int BN>
hipError_t launch(hipStream_t stream, const PrepareArgs &p, const gemm::GemmArgs &g, int cus,
                  unsigned int *state) {
  const int tiles = ((g.m + BM - 1) / BM) * (g.n / BN);
  hipLaunchKernelGGL(reset_kernel, dim3(1), dim3(kStateBytes / 4), 0, stream, state);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds = lds_bytes<kKind, BM, BN>(p.width);
  hipLaunchKernelGGL((prepare_gemm_kernel<kKind, T, BM, BN>), dim3(cus), dim3(512), lds, stream, p, g, tiles,
                     state, barrier_polls());
  return hipGetLastError();
}

}  // namespace fused

hipError_t configure_fused_lds() { return fused::configure(); }

// The fused launch for whole rounds of 256x192 tiles (the tile choice of launch_gemm
// for QKV-like shapes); hipErrorNotSupported for every other shape, and for a stream
// without a workspace (a capture with none installed or registered), which the caller
// then runs as two launches. The barrier's state is the first bytes of the stream's
// workspace: calls on one stream are ordered, and calls on different streams use
// different workspaces, so every launch has its own. (256x256 tiles do not fit the
// prepare's registers beside the tile's: they would spill.)
hipError_t launch_prepare_gemm(int kind, hipStream_t stream, int64_t tokens,
                               const PrepareLaunch &pl, const GemmLaunch &gl) {
  const int cus = device_cus();
  if (!one_launch_fits(tokens, gl.m, gl.n, pl.width, gl.lda, pl.out_stride, cus)) return hipErrorNotSupported;
  const Workspace ws = gl.workspace ? *gl.workspace : splitk_workspace(stream);
  if (!ws.ptr || ws.bytes < fused::kStateBytes) return hipErrorNotSupported;
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
  unsigned int *state = static_cast<unsigned int *>(ws.ptr);
  const int t = (int)((pl.width / 16 + 63) / 64);  // runs of 16 per lane
  if (kind == kNorm)
    return t <= 2 ? fused::launch<kNorm, 2, 256, 192>(stream, p, g, cus, state)
                  : fused::launch<kNorm, 3, 256, 192>(stream, p, g, cus, state);
  return t <= 2 ? fused::launch<kPlain, 2, 256, 192>(stream, p, g, cus, state)
                : fused::launch<kPlain, 3, 256, 192>(stream, p, g, cus, state);
}

}  // namespace k2w8
