// INT8 GEMM family for few tokens (the text-encoder-shaped regime, M <= 64 per token
// group), where the weights dominate HBM traffic and the MFMAs are nearly idle.
//
// One workgroup owns RB weight rows (16 or 32: a SwiGLU gate|up pair) and a group of
// up to 64 tokens (TB blocks of 16). Its WAVES waves split K into contiguous ranges;
// each wave streams its range of the weight rows and token rows straight from global
// memory into registers (no LDS staging: every weight byte is used by one MFMA per
// token block), keeping several 64-byte K steps in flight while it computes on
// v_mfma_i32_16x16x64_i8. The waves' int32 partial sums meet in LDS (integer
// addition: the order is irrelevant, the result exact), and each wave then runs the
// dequantising epilogue for one token block.
//
// Each 64-byte K step is one MFMA per (row block, token block): lane (r, kq) supplies
// bytes [16 kq, 16 kq + 16) of row r for both operands.
//
// Results are identical to the large-tile kernels' (same int32 accumulators, same
// epilogue arithmetic): kernels/gemm_i8_256.loom:606-626 and its residual and SwiGLU
// siblings.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Epilogue of one 16-token block. With the weights as the MFMA row operand, lane
// (t, kq) holds token t0 + t and, in register e, channel n0 + 16 rb + 4 kq + e.
template <int EPI, int RB>
__device__ __forceinline__ void store_block(const Args &g, const v4i (&acc)[RB / 16], int n0, int tok,
                                            int kq) {
  if (tok >= g.m) return;
  const float as = (EPI == kEpiAcc) ? 1.0f : g.a_scale[tok];
  if (EPI == kEpiSwiglu) {
    // rb 0: gate channels n0 + 4kq + e; rb 1: the matching ups, 16 rows further on.
    const float4 gs = *reinterpret_cast<const float4 *>(g.w_scale + n0 + 4 * kq);
    const float4 us = *reinterpret_cast<const float4 *>(g.w_scale + n0 + 16 + 4 * kq);
    const float gsv[4] = {gs.x, gs.y, gs.z, gs.w}, usv[4] = {us.x, us.y, us.z, us.w};
    uint32_t packed[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      float g0 = ((float)acc[0][e] * gsv[e]) * as, g1 = ((float)acc[0][e + 1] * gsv[e + 1]) * as;
      float u0 = ((float)acc[RB / 16 - 1][e] * usv[e]) * as;
      float u1 = ((float)acc[RB / 16 - 1][e + 1] * usv[e + 1]) * as;
      bf16_round2(g0, g1);
      bf16_round2(u0, u1);
      float s0 = g0 * sigmoid(g0), s1 = g1 * sigmoid(g1);
      bf16_round2(s0, s1);
      float p0 = s0 * u0, p1 = s1 * u1;
      bf16_round2(p0, p1);
      packed[e >> 1] = f16_pack2(p0, p1);
    }
    uint16_t *out = static_cast<uint16_t *>(g.c) + (int64_t)tok * (g.n >> 1) + (n0 >> 1) + 4 * kq;
    *reinterpret_cast<uint2 *>(out) = make_uint2(packed[0], packed[1]);
    return;
  }
#pragma unroll
  for (int rb = 0; rb < RB / 16; ++rb) {
    const int nb = n0 + 16 * rb + 4 * kq;
    if (EPI == kEpiAcc) {
      *reinterpret_cast<v4i *>(static_cast<int32_t *>(g.c) + (int64_t)tok * g.n + nb) = acc[rb];
      continue;
    }
    const float4 ws4 = *reinterpret_cast<const float4 *>(g.w_scale + nb);
    const float ws[4] = {ws4.x, ws4.y, ws4.z, ws4.w};
    float extra[4] = {0.f, 0.f, 0.f, 0.f};
    if (EPI == kEpiResid) {
      const float4 v = *reinterpret_cast<const float4 *>(g.gate + nb);
      extra[0] = v.x; extra[1] = v.y; extra[2] = v.z; extra[3] = v.w;
    }
    if (EPI == kEpiBias) {
      const uint2 v = *reinterpret_cast<const uint2 *>(g.bias + nb);
      extra[0] = f16_value(v.x & 0xffffu); extra[1] = f16_value(v.x >> 16);
      extra[2] = f16_value(v.y & 0xffffu); extra[3] = f16_value(v.y >> 16);
    }
    uint16_t *out = static_cast<uint16_t *>(g.c) + (int64_t)tok * g.n + nb;
    uint2 prior = make_uint2(0, 0);
    if (EPI == kEpiResid) prior = *reinterpret_cast<const uint2 *>(out);
    const uint32_t pw[2] = {prior.x, prior.y};
    uint32_t packed[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      float v0 = ((float)acc[rb][e] * ws[e]) * as, v1 = ((float)acc[rb][e + 1] * ws[e + 1]) * as;
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
    *reinterpret_cast<uint2 *>(out) = make_uint2(packed[0], packed[1]);
  }
}

template <int RB, int TB, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES * 64) void skinny_kernel(Args g) {
  __shared__ v4i partial[WAVES][RB / 16][TB][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int n0 = blockIdx.x * RB;
  const int t0 = blockIdx.y * kTokensPerGroup;

  // This wave's K range, in 64-byte steps; lane (r, kq) loads bytes [16 kq, 16 kq + 16)
  // of each step for its weight rows and token rows.
  const int steps = g.k >> 6;
  const int s_lo = steps * wave / WAVES, s_hi = steps * (wave + 1) / WAVES;
  const int count = s_hi - s_lo;

  const int8_t *wrow[RB / 16];
  const int8_t *arow[TB];
#pragma unroll
  for (int rb = 0; rb < RB / 16; ++rb)
    wrow[rb] = g.w + (int64_t)(n0 + 16 * rb + r) * g.lda + s_lo * 64 + kq * 16;
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
    arow[tb] = g.a + (int64_t)min(t0 + 16 * tb + r, g.m - 1) * g.lda + s_lo * 64 + kq * 16;

  v4i acc[RB / 16][TB];
#pragma unroll
  for (int rb = 0; rb < RB / 16; ++rb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[rb][tb] = v4i{0, 0, 0, 0};

  // A ring of P steps in flight: the loads of step i+P are issued as step i computes,
  // so each wave keeps P steps of its rows outstanding (the weights stream from HBM).
  constexpr int P = (RB / 16 + TB) <= 3 ? 8 : 4;
  v4i wf[P][RB / 16], af[P][TB];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    if (p < count) {
#pragma unroll
      for (int rb = 0; rb < RB / 16; ++rb) wf[p][rb] = *reinterpret_cast<const v4i *>(wrow[rb] + p * 64);
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) af[p][tb] = *reinterpret_cast<const v4i *>(arow[tb] + p * 64);
    }
  }
  for (int base = 0; base < count; base += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int st = base + p;
      if (st < count) {
#pragma unroll
        for (int rb = 0; rb < RB / 16; ++rb)
#pragma unroll
          for (int tb = 0; tb < TB; ++tb)
            acc[rb][tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[p][rb], af[p][tb], acc[rb][tb], 0, 0, 0);
        if (st + P < count) {
#pragma unroll
          for (int rb = 0; rb < RB / 16; ++rb)
            wf[p][rb] = *reinterpret_cast<const v4i *>(wrow[rb] + (st + P) * 64);
#pragma unroll
          for (int tb = 0; tb < TB; ++tb)
            af[p][tb] = *reinterpret_cast<const v4i *>(arow[tb] + (st + P) * 64);
        }
      }
    }
  }

  // Combine the waves' partial sums; wave w finishes token block w.
#pragma unroll
  for (int rb = 0; rb < RB / 16; ++rb)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) partial[wave][rb][tb][lane] = acc[rb][tb];
  __syncthreads();
  if (wave < TB) {
    v4i sum[RB / 16];
#pragma unroll
    for (int rb = 0; rb < RB / 16; ++rb) {
      sum[rb] = partial[0][rb][wave][lane];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum[rb] += partial[w][rb][wave][lane];
    }
    store_block<EPI, RB>(g, sum, n0, t0 + 16 * wave + r, kq);
  }
}

template <int RB, int TB, int WAVES>
hipError_t launch_rb(int epi, hipStream_t stream, const Args &a) {
  dim3 grid(a.n / RB, (a.m + kTokensPerGroup - 1) / kTokensPerGroup), block(WAVES * 64);
  switch (epi) {
    case kEpiPlain: hipLaunchKernelGGL((skinny_kernel<RB, TB, WAVES, kEpiPlain>), grid, block, 0, stream, a); break;
    case kEpiResid: hipLaunchKernelGGL((skinny_kernel<RB, TB, WAVES, kEpiResid>), grid, block, 0, stream, a); break;
    case kEpiSwiglu: hipLaunchKernelGGL((skinny_kernel<RB, TB, WAVES, kEpiSwiglu>), grid, block, 0, stream, a); break;
    case kEpiBias: hipLaunchKernelGGL((skinny_kernel<RB, TB, WAVES, kEpiBias>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((skinny_kernel<RB, TB, WAVES, kEpiAcc>), grid, block, 0, stream, a); break;
  }
  return hipGetLastError();
}

template <int TB>
hipError_t launch_tb(int epi, hipStream_t stream, const Args &a) {
  if (epi == kEpiSwiglu) return launch_rb<32, TB, 4>(epi, stream, a);
  return launch_rb<16, TB, 4>(epi, stream, a);
}

}  // namespace skinny

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
  switch ((tokens + 15) / 16) {
    case 1: return skinny::launch_tb<1>(epilogue, stream, a);
    case 2: return skinny::launch_tb<2>(epilogue, stream, a);
    case 3: return skinny::launch_tb<3>(epilogue, stream, a);
    default: return skinny::launch_tb<4>(epilogue, stream, a);
  }
}

}  // namespace k2w8
