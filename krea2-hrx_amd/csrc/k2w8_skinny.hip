// INT8 GEMM family for few tokens (the text-encoder-shaped regime, M <= 64 per token
// group), where the weights dominate HBM traffic and the MFMAs are nearly idle.
//
// One workgroup owns RB weight rows (16, or 32: a SwiGLU gate|up pair) and a group of
// up to 64 tokens (TB blocks of 16). Its waves split K into contiguous ranges; each
// wave streams its range of weight and token rows global -> LDS through a ring of its
// own (several 128-byte K steps in flight, every transfer whole cache lines) and reads
// the fragments of v_mfma_i32_16x16x64_i8 back from it. The waves' int32 partial sums
// meet in LDS (integer addition: the order is irrelevant, the result exact), and wave w
// runs the dequantising epilogue for token block w.
//
// Each 64-byte half of a K step is one MFMA per (row block, token block): lane (r, kq)
// supplies bytes [16 kq, 16 kq + 16) of row r for both operands.
//
// Results are identical to the large-tile kernels' (same int32 accumulators, same
// epilogue arithmetic): kernels/gemm_i8_256.loom:606-626 and its residual and SwiGLU
// siblings.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k2w8_gemm_common.hpp"
#include "k2w8_internal.hpp"
#include "k2w8_numerics.hpp"

namespace k2w8 {
namespace skinny {

typedef int v4i __attribute__((ext_vector_type(4)));

struct Args {
  const int8_t *a, *w;
  const float *w_scale, *a_scale;
  void *c;
  const float *gate;
  const uint16_t *bias;
  int m, n, k, lda;
};

constexpr int kTokensPerGroup = 64;

// The weight and token rows go global -> LDS through a per-wave ring of P 128-byte K
// steps (global_load_lds_dwordx4), each transfer instruction covering 8 rows x 128
// bytes, i.e. whole cache lines: measured on a plain read of the QKV weights, 16 rows
// x 64 bytes per instruction (the MFMA register layout, loaded directly) took 4.3 us
// and whole lines 3.5 us.
// Each wave owns its ring, so the K loop needs no workgroup barrier. The epilogue's
// per-channel and per-token operands are loaded before the K loop, so their latency
// hides behind the weight stream instead of following it.
template <int RB>
struct Rows {
  static_assert(RB % 16 == 0, "whole 16-row MFMA blocks");
  static constexpr int kBlocks = RB / 16;  // 16-row MFMA blocks
  static constexpr int kLoads = RB / 8;    // 8-row transfers per step
};

// Chunk swizzle of a staged 128-byte row (as in the tile kernels): 16-byte chunk c of
// row r sits at position c ^ key(r), so one LDS cycle's rows spread over the banks.
__device__ __forceinline__ int skey(int r) { return (r >> 1) & 7; }

template <int P, int I>
__device__ __forceinline__ void wait_steps(int newer) {
  // Wait until at most `newer` steps (I transfers each) are still in flight.
  if (newer >= P - 1) { gemm::wait_vmcnt<(P - 1) * I>(); return; }
  switch (newer) {
    case 0: gemm::wait_vmcnt<0>(); break;
    case 1: gemm::wait_vmcnt<(P > 1 ? 1 : 0) * I>(); break;
    case 2: gemm::wait_vmcnt<(P > 2 ? 2 : 0) * I>(); break;
    case 3: gemm::wait_vmcnt<(P > 3 ? 3 : 0) * I>(); break;
    case 4: gemm::wait_vmcnt<(P > 4 ? 4 : 0) * I>(); break;
    case 5: gemm::wait_vmcnt<(P > 5 ? 5 : 0) * I>(); break;
    case 6: gemm::wait_vmcnt<(P > 6 ? 6 : 0) * I>(); break;
    default: gemm::wait_vmcnt<0>(); break;
  }
}

// AR: token rows staged per token block, 16, or 8 for at most 8 tokens (MFMA columns
// 8-15 then repeat columns 0-7 and are not stored).
template <int TB, int AR>
constexpr int token_loads() { return TB * AR / 8; }

template <int RB, int TB, int AR, int WAVES, int P, int EPI>
__global__ __launch_bounds__(WAVES * 64) void stream_kernel(Args g) {
  static_assert(P >= 2 && P <= 8, "ring depth");
  static_assert(AR == 16 || (AR == 8 && TB == 1), "token rows");
  constexpr int RBK = Rows<RB>::kBlocks, WL = Rows<RB>::kLoads;
  constexpr int I = WL + token_loads<TB, AR>();  // transfers per step: weights, then tokens
  constexpr int kStep = I * 1024;      // LDS bytes per step
  constexpr int kA = WL * 1024;        // token rows' offset within a step
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int n0 = blockIdx.x * RB;
  const int t0 = blockIdx.y * kTokensPerGroup;

  // SwiGLU over the interleaved 32-row groups [gate o..o+15 | up o..o+15]: with RB=32
  // a workgroup takes a whole group (rb 0 gates, rb 1 ups); with RB=16 it takes half of
  // one, 8 gate rows and their 8 up rows (half j = blockIdx.x & 1 of group
  // blockIdx.x >> 1). Staged rows 0-7 are then the gates, 8-15 the ups, so lanes kq < 2
  // end with the gates' sums and lanes kq >= 2 with the ups' (exchanged across lane
  // halves for the epilogue).
  constexpr bool kPairRows = EPI == kEpiSwiglu && RB == 16;
  static_assert(EPI != kEpiSwiglu || RB == 16 || RB == 32, "SwiGLU workgroup rows");
  const int gate0 = 32 * (blockIdx.x >> 1) + 8 * (blockIdx.x & 1), up0 = gate0 + 16;

  // Epilogue operands, loaded now. Lane (r, kq) of wave w < TB finishes token
  // t0 + 16w + r, channels n0 + 16 rb + 4 kq + e (SwiGLU: gate channels gate0 + 4 kq + e
  // and the matching ups, lanes kq < 2).
  const int tok = t0 + 16 * wave + r;
  const bool stores = wave < TB && tok < g.m && (AR == 16 || r < 8) && (!kPairRows || kq < 2);
  float4 ws[RBK], gs[RBK];
  uint2 prior[RBK], bias[RBK];
  float as = 0.0f;
  if (stores) {
    as = (EPI == kEpiAcc) ? 1.0f : g.a_scale[tok];
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb) {
      const int nb = n0 + 16 * rb + 4 * kq;
      if (kPairRows) {
        ws[rb] = *reinterpret_cast<const float4 *>(g.w_scale + gate0 + 4 * kq);
        gs[rb] = *reinterpret_cast<const float4 *>(g.w_scale + up0 + 4 * kq);
        continue;
      }
      if (EPI != kEpiAcc) ws[rb] = *reinterpret_cast<const float4 *>(g.w_scale + nb);
      if (EPI == kEpiResid) {
        gs[rb] = *reinterpret_cast<const float4 *>(g.gate + nb);
        prior[rb] = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(g.c) + (int64_t)tok * g.n + nb);
      }
      if (EPI == kEpiBias) bias[rb] = *reinterpret_cast<const uint2 *>(g.bias + nb);
    }
  }

  // This wave's K range in 128-byte steps.
  const int steps = g.k >> 7;
  const int lo = steps * wave / WAVES, hi = steps * (wave + 1) / WAVES;
  const int count = hi - lo;
  const uint32_t ring = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)) + wave * (P * kStep);

  // Transfer i of a step covers 8 staged rows: weights (i < WL), then token rows.
  // Lane l brings logical chunk (l & 7) ^ key(row) of row (l >> 3), so staged position
  // l & 7 holds it.
  uint32_t off[I];
  const int8_t *src[I];
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int row = (i < WL ? 8 * i : 8 * (i - WL)) + (lane >> 3);
    const int c = (lane & 7) ^ skey(row);
    if (i < WL) {
      src[i] = g.w;
      const int wrow = kPairRows ? (i == 0 ? gate0 : up0) + (lane >> 3) : n0 + row;
      off[i] = (uint32_t)wrow * (uint32_t)g.lda + lo * 128 + c * 16;
    } else {
      src[i] = g.a;
      off[i] = (uint32_t)min(t0 + row, g.m - 1) * (uint32_t)g.lda + lo * 128 + c * 16;
    }
  }
  auto issue = [&](int st) {  // step lo + st into slot st % P
    const uint32_t base = ring + (uint32_t)((st % P) * kStep);
#pragma unroll
    for (int i = 0; i < I; ++i) gemm::dma16(base + i * 1024, src[i], off[i] + st * 128);
  };
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (p < count) issue(p);

  // Fragment offsets within a step: row block rb, token block tb, K half h, chunk kq.
  int w_off[RBK][2], a_off[TB][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb) {
      const int row = 16 * rb + r;
      w_off[rb][h] = row * 128 + (((4 * h + kq) ^ skey(row)) << 4);
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int row = AR == 16 ? 16 * tb + r : (r & 7);
      a_off[tb][h] = kA + row * 128 + (((4 * h + kq) ^ skey(row)) << 4);
    }
  }

  v4i acc[RBK][TB];
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[rb][tb] = v4i{0, 0, 0, 0};

  for (int st = 0; st < count; ++st) {
    wait_steps<P, I>(min(count - 1 - st, P - 1));
    const uint8_t *slot = smem + wave * (P * kStep) + (st % P) * kStep;
    v4i wf[2][RBK], af[2][TB];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb) wf[h][rb] = *reinterpret_cast<const v4i *>(slot + w_off[rb][h]);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) af[h][tb] = *reinterpret_cast<const v4i *>(slot + a_off[tb][h]);
    }
    // The slot is free once these reads have returned: refill it with step st + P.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (st + P < count) issue(st + P);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
          acc[rb][tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[h][rb], af[h][tb], acc[rb][tb], 0, 0, 0);
  }

  // Combine the waves' partial sums (the rings are done: reuse their LDS); wave w
  // finishes token block w.
  __syncthreads();
  v4i *partial = reinterpret_cast<v4i *>(smem);  // [WAVES][RBK][TB][64]
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) partial[((wave * RBK + rb) * TB + tb) * 64 + lane] = acc[rb][tb];
  __syncthreads();
  if (wave >= TB) return;
  v4i sum[RBK];
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb) {
    sum[rb] = partial[(rb * TB + wave) * 64 + lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum[rb] += partial[((w * RBK + rb) * TB + wave) * 64 + lane];
  }
  v4i pair_up{};
  if (kPairRows) {
    // The ups' sums, from lane l + 32 (every lane of the wave takes part in the swap).
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const auto sw = __builtin_amdgcn_permlane32_swap((uint32_t)sum[0][e], (uint32_t)sum[0][e], false, false);
      pair_up[e] = (int)sw[1];
    }
  }
  if (!stores) return;
  if (EPI == kEpiSwiglu) {
    const float gsv[4] = {ws[0].x, ws[0].y, ws[0].z, ws[0].w};
    const float4 us = kPairRows ? gs[0] : ws[RBK - 1];
    const float usv[4] = {us.x, us.y, us.z, us.w};
    const v4i gate = sum[0], up = kPairRows ? pair_up : sum[RBK - 1];
    float gv[4], uv[4];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      float g0 = ((float)gate[e] * gsv[e]) * as, g1 = ((float)gate[e + 1] * gsv[e + 1]) * as;
      float u0 = ((float)up[e] * usv[e]) * as;
      float u1 = ((float)up[e + 1] * usv[e + 1]) * as;
      bf16_round2(g0, g1);
      bf16_round2(u0, u1);
      gv[e] = g0; gv[e + 1] = g1; uv[e] = u0; uv[e + 1] = u1;
    }
    swiglu_products(gv, uv);
    const uint32_t packed[2] = {f16_pack2(gv[0], gv[1]), f16_pack2(gv[2], gv[3])};
    const int col = kPairRows ? 16 * (blockIdx.x >> 1) + 8 * (blockIdx.x & 1) : n0 >> 1;
    uint16_t *out = static_cast<uint16_t *>(g.c) + (int64_t)tok * (g.n >> 1) + col + 4 * kq;
    *reinterpret_cast<uint2 *>(out) = make_uint2(packed[0], packed[1]);
    return;
  }
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb) {
    const int nb = n0 + 16 * rb + 4 * kq;
    if (EPI == kEpiAcc) {
      *reinterpret_cast<v4i *>(static_cast<int32_t *>(g.c) + (int64_t)tok * g.n + nb) = sum[rb];
      continue;
    }
    const float wsv[4] = {ws[rb].x, ws[rb].y, ws[rb].z, ws[rb].w};
    float extra[4] = {0.f, 0.f, 0.f, 0.f};
    if (EPI == kEpiResid) {
      extra[0] = gs[rb].x; extra[1] = gs[rb].y; extra[2] = gs[rb].z; extra[3] = gs[rb].w;
    }
    if (EPI == kEpiBias) {
      extra[0] = f16_value(bias[rb].x & 0xffffu); extra[1] = f16_value(bias[rb].x >> 16);
      extra[2] = f16_value(bias[rb].y & 0xffffu); extra[3] = f16_value(bias[rb].y >> 16);
    }
    const uint32_t pw[2] = {EPI == kEpiResid ? prior[rb].x : 0u, EPI == kEpiResid ? prior[rb].y : 0u};
    uint32_t packed[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      float v0 = ((float)sum[rb][e] * wsv[e]) * as, v1 = ((float)sum[rb][e + 1] * wsv[e + 1]) * as;
      if (EPI == kEpiBias) {
        v0 = v0 + extra[e];
        v1 = v1 + extra[e + 1];
      }
      bf16_round2(v0, v1);
      if (EPI == kEpiResid) {  // x = bf16(x + bf16(gate * bf16(v)))
        float g0 = v0 * extra[e], g1 = v1 * extra[e + 1];
        bf16_round2(g0, g1);
        const uint32_t w = pw[e >> 1];
        packed[e >> 1] = bf16_pack2(__uint_as_float(w << 16) + g0, __uint_as_float(w & 0xffff0000u) + g1);
      } else {
        packed[e >> 1] = f16_pack2(v0, v1);
      }
    }
    uint16_t *out = static_cast<uint16_t *>(g.c) + (int64_t)tok * g.n + nb;
    *reinterpret_cast<uint2 *>(out) = make_uint2(packed[0], packed[1]);
  }
}

template <int RB, int TB, int AR, int WAVES, int P>
struct StreamConfig {
  static constexpr size_t kLds = (size_t)WAVES * P * (Rows<RB>::kLoads + token_loads<TB, AR>()) * 1024;
};

template <int RB, int TB, int AR, int WAVES, int P>
hipError_t launch_stream(int epi, hipStream_t stream, const Args &a) {
  constexpr size_t lds = StreamConfig<RB, TB, AR, WAVES, P>::kLds;
  static_assert(lds <= 160 * 1024, "LDS");
  dim3 grid(a.n / RB, (a.m + kTokensPerGroup - 1) / kTokensPerGroup), block(WAVES * 64);
  switch (epi) {
    case kEpiPlain: hipLaunchKernelGGL((stream_kernel<RB, TB, AR, WAVES, P, kEpiPlain>), grid, block, lds, stream, a); break;
    case kEpiResid: hipLaunchKernelGGL((stream_kernel<RB, TB, AR, WAVES, P, kEpiResid>), grid, block, lds, stream, a); break;
    case kEpiSwiglu: hipLaunchKernelGGL((stream_kernel<RB, TB, AR, WAVES, P, kEpiSwiglu>), grid, block, lds, stream, a); break;
    case kEpiBias: hipLaunchKernelGGL((stream_kernel<RB, TB, AR, WAVES, P, kEpiBias>), grid, block, lds, stream, a); break;
    default: hipLaunchKernelGGL((stream_kernel<RB, TB, AR, WAVES, P, kEpiAcc>), grid, block, lds, stream, a); break;
  }
  return hipGetLastError();
}

template <int RB, int TB, int AR, int WAVES, int P>
hipError_t set_lds_stream() {
  constexpr size_t lds = StreamConfig<RB, TB, AR, WAVES, P>::kLds;
  const void *fns[5] = {reinterpret_cast<const void *>(stream_kernel<RB, TB, AR, WAVES, P, kEpiPlain>),
                        reinterpret_cast<const void *>(stream_kernel<RB, TB, AR, WAVES, P, kEpiResid>),
                        reinterpret_cast<const void *>(stream_kernel<RB, TB, AR, WAVES, P, kEpiSwiglu>),
                        reinterpret_cast<const void *>(stream_kernel<RB, TB, AR, WAVES, P, kEpiBias>),
                        reinterpret_cast<const void *>(stream_kernel<RB, TB, AR, WAVES, P, kEpiAcc>)};
  for (const void *f : fns) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// LDS budget of a workgroup's rings (KiB), and the deepest ring.
constexpr int kRingKb = 48, kRingMax = 8;

// Ring depth: as many steps as fit the LDS budget per workgroup (at least 2).
constexpr int ring_depth_of(int rb, int tb, int ar, int waves) {
  const int per_step = waves * (rb / 8 + tb * ar / 8);  // KiB
  const int p = kRingKb / per_step;
  return p < 2 ? 2 : (p > kRingMax ? kRingMax : p);
}

// Workgroup shape: 16 rows, or for SwiGLU a whole gate|up group (32 rows) when 16
// token rows are staged and half of one (8 gates, their 8 ups) when 8 are; four waves, or
// eight when N/16 workgroups would leave CUs idle (each wave then streams half as
// many K steps). Measured on the down projection (N=2560, K=9728) against 8-row
// workgroups of four waves: M=1 7.9 -> 6.8 us, M=16 11.1 -> 8.9, M=32 15.7 -> 11.3.
// Half groups double the SwiGLU workgroups (N=19456: 608 -> 1216 on 256 CUs), which
// evens out the last round: up projection at K=2560, M=1 11.3 -> 10.7 us, M=8 11.6 ->
// 10.8. With 16 token rows each workgroup stages as many token bytes as weight bytes,
// and twice the workgroups cost more than they even out (M=16 12.3 -> 12.7, M=32 14.0
// -> 16.2), so there the workgroups keep whole groups.
int rows_of(int epi, int ar) { return epi == kEpiSwiglu && ar == 16 ? 32 : 16; }
int waves_of(int epi, int64_t n, int64_t cus) { return epi != kEpiSwiglu && n / 16 < cus ? 8 : 4; }

template <int RB, int TB, int AR, int WAVES>
hipError_t launch_rows(int epi, hipStream_t stream, const Args &a) {
  return launch_stream<RB, TB, AR, WAVES, ring_depth_of(RB, TB, AR, WAVES)>(epi, stream, a);
}

template <int TB, int AR>
hipError_t launch_tb(int epi, hipStream_t stream, const Args &a) {
  if constexpr (AR == 16)
    if (epi == kEpiSwiglu) return launch_rows<32, TB, AR, 4>(epi, stream, a);
  if (waves_of(epi, a.n, device_cus()) == 8) return launch_rows<16, TB, AR, 8>(epi, stream, a);
  return launch_rows<16, TB, AR, 4>(epi, stream, a);
}

template <int TB, int AR>
hipError_t set_lds_tb() {
  hipError_t e = set_lds_stream<16, TB, AR, 4, ring_depth_of(16, TB, AR, 4)>();
  if (e == hipSuccess) e = set_lds_stream<16, TB, AR, 8, ring_depth_of(16, TB, AR, 8)>();
  if constexpr (AR == 16)
    if (e == hipSuccess) e = set_lds_stream<32, TB, AR, 4, ring_depth_of(32, TB, AR, 4)>();
  return e;
}

}  // namespace skinny

// Past kSkinnyMaxTokens the streaming kernel still wins while K is short and its
// grid (one workgroup per RB weight rows and per 64 tokens) is resident at once:
// measured at K=2560, N=4096, M=64-128: 12-15 -> 7-9 us; where the grid takes two
// rounds (N=19456, M=64) or K is long (9728), the tile kernels are faster.
bool skinny_streams(int epilogue, const GemmLaunch &l, int64_t cus) {
  if (l.m > 128 || l.k > 4096) return false;
  const int64_t tokens = l.m < skinny::kTokensPerGroup ? l.m : skinny::kTokensPerGroup;
  const int tb = (int)((tokens + 15) / 16), ar = tokens <= 8 ? 8 : 16;
  const int rb = skinny::rows_of(epilogue, ar), waves = skinny::waves_of(epilogue, l.n, cus);
  const int lds_kb = waves * skinny::ring_depth_of(rb, tb, ar, waves) * (rb / 8 + tb * ar / 8);
  const int64_t per_cu = 160 / lds_kb;
  const int64_t grid = (l.n / rb) * ((l.m + skinny::kTokensPerGroup - 1) / skinny::kTokensPerGroup);
  return grid <= per_cu * cus;
}

hipError_t configure_skinny_lds() {
  hipError_t e = skinny::set_lds_tb<1, 8>();
  if (e == hipSuccess) e = skinny::set_lds_tb<1, 16>();
  if (e == hipSuccess) e = skinny::set_lds_tb<2, 16>();
  if (e == hipSuccess) e = skinny::set_lds_tb<3, 16>();
  if (e == hipSuccess) e = skinny::set_lds_tb<4, 16>();
  return e;
}

hipError_t launch_skinny(int epilogue, hipStream_t stream, const GemmLaunch &l) {
  skinny::Args a;
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
  const int tokens = (int)(l.m < skinny::kTokensPerGroup ? l.m : skinny::kTokensPerGroup);
  if (tokens <= 8) return skinny::launch_tb<1, 8>(epilogue, stream, a);
  switch ((tokens + 15) / 16) {
    case 1: return skinny::launch_tb<1, 16>(epilogue, stream, a);
    case 2: return skinny::launch_tb<2, 16>(epilogue, stream, a);
    case 3: return skinny::launch_tb<3, 16>(epilogue, stream, a);
    default: return skinny::launch_tb<4, 16>(epilogue, stream, a);
  }
}

}  // namespace k2w8
