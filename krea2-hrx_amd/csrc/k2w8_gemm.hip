// INT8 GEMM family of the W8A8 path for gfx950 (CDNA4):
//   acc[m][n] = sum_k A[m][k] * W[n][k]   (exact int32, v_mfma_i32_32x32x32_i8)
// followed by a fused dequantising epilogue (plain f16, bf16 gated residual in
// place, SwiGLU, plain + bias, or the raw int32 accumulators).
//
// Workgroup tile BM x BN with a 128-byte K step; both operands are K-contiguous
// rows, staged through LDS in a 16-byte-chunk XOR swizzle and double buffered:
// the next K step's global loads are in flight while the current step's MFMAs
// run, and each wave reads the next 32-byte K slice's fragments from LDS while
// the current slice's MFMAs issue. Each wave64 owns a (BM/WM) x (BN/WN) sub-tile
// of 32x32 MFMA blocks. Workgroups are numbered XCD-major (consecutive tiles land
// on one XCD's L2), then grouped m_group m-tiles per sweep of n.
//
// Reference: kernels/gemm_i8_256.loom (tile, raster groups :98-132, ghost rows
// :169-216, epilogue :558-629), kernels/gemm_i8_resid_256.loom:607-635,
// kernels/gemm_i8_swiglu_256.loom:569-660.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "k2w8_gemm_common.hpp"
#include "k2w8_gemm_plan.hpp"
#include "k2w8_internal.hpp"
#include "k2w8_numerics.hpp"

namespace k2w8 {

namespace gemm {

typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
// Buffer descriptor word 3 for raw 32-bit buffer access on CDNA (no swizzle, no format
// conversion), and the cache-policy operand bit of a store's sc1 (system coherence scope:
// the L2 writes the data through).
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCachePolicySc1 = 16;

// Epilogue of one wave's (32 FM) x (32 FN) sub-tile at rows m_base.., columns n_base..
template <int EPI, int FM, int FN>
__device__ __forceinline__ void store_tile(const GemmArgs &g, int split, v16i (&acc)[FM][FN], int m_base,
                                           int n_base, int fr, int kh) {
  // The MFMAs run with the weights as their row operand, so block (i, j) holds C^T:
  // lane (fr, kh) owns token m = m_base + 32i + fr and, in register e, channel
  // n = n_base + 32j + 8(e/4) + 4kh + e%4. Each lane therefore holds
  // four runs of four consecutive channels of one token: 8-byte f16 / bf16 stores.
  int64_t m_row[FM];
  float as[FM];
  bool live[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m_base + i * 32 + fr;
    live[i] = m < g.m;
    m_row[i] = live[i] ? m : g.m - 1;
    as[i] = (EPI == kEpiAcc) ? 1.0f : g.a_scale[m_row[i]];
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int nb = n_base + j * 32 + kh * 4;  // channel of register 0
    if (EPI == kEpiSwiglu) {
      // registers 0-7: gate channels 8q+4kh+r (q<2) of the 32-channel group,
      // registers 8-15: the matching up channels, 16 further on
      float4 wg[2], wu[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        wg[q] = *reinterpret_cast<const float4 *>(g.w_scale + nb + 8 * q);
        wu[q] = *reinterpret_cast<const float4 *>(g.w_scale + nb + 16 + 8 * q);
      }
      const int ob = ((n_base + j * 32) >> 1) + kh * 4;  // output of register 0
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (!live[i]) continue;
        uint16_t *out = static_cast<uint16_t *>(g.c) + m_row[i] * g.ldc + ob;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float gs[4] = {wg[q].x, wg[q].y, wg[q].z, wg[q].w};
          const float us[4] = {wu[q].x, wu[q].y, wu[q].z, wu[q].w};
          uint32_t packed[2];
#pragma unroll
          for (int r = 0; r < 4; r += 2) {
            float g0 = ((float)acc[i][j][4 * q + r] * gs[r]) * as[i];
            float g1 = ((float)acc[i][j][4 * q + r + 1] * gs[r + 1]) * as[i];
            float u0 = ((float)acc[i][j][8 + 4 * q + r] * us[r]) * as[i];
            float u1 = ((float)acc[i][j][8 + 4 * q + r + 1] * us[r + 1]) * as[i];
            bf16_round2(g0, g1);
            bf16_round2(u0, u1);
            float s0 = g0 * sigmoid(g0), s1 = g1 * sigmoid(g1);
            bf16_round2(s0, s1);
            float p0 = s0 * u0, p1 = s1 * u1;
            bf16_round2(p0, p1);
            packed[r >> 1] = f16_pack2(p0, p1);
          }
          *reinterpret_cast<uint2 *>(out + 8 * q) = make_uint2(packed[0], packed[1]);
        }
      }
      continue;
    }
    float ws[16], extra[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (EPI != kEpiAcc) {
        const float4 v = *reinterpret_cast<const float4 *>(g.w_scale + nb + 8 * q);
        ws[4 * q] = v.x; ws[4 * q + 1] = v.y; ws[4 * q + 2] = v.z; ws[4 * q + 3] = v.w;
      }
      if (EPI == kEpiResid) {
        const float4 v = *reinterpret_cast<const float4 *>(g.gate + nb + 8 * q);
        extra[4 * q] = v.x; extra[4 * q + 1] = v.y; extra[4 * q + 2] = v.z; extra[4 * q + 3] = v.w;
      }
      if (EPI == kEpiBias) {
        const uint2 v = *reinterpret_cast<const uint2 *>(g.bias + nb + 8 * q);
        extra[4 * q] = f16_value(v.x & 0xffffu); extra[4 * q + 1] = f16_value(v.x >> 16);
        extra[4 * q + 2] = f16_value(v.y & 0xffffu); extra[4 * q + 3] = f16_value(v.y >> 16);
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (!live[i]) continue;
      if (EPI == kEpiAcc) {
        int32_t *out = static_cast<int32_t *>(g.c) + (int64_t)split * g.split_stride +
                       m_row[i] * g.ldc + nb;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<v4i *>(out + 8 * q) =
              v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        continue;
      }
      uint16_t *out = static_cast<uint16_t *>(g.c) + m_row[i] * g.ldc + nb;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint2 prior = make_uint2(0, 0);
        if (EPI == kEpiResid) prior = *reinterpret_cast<const uint2 *>(out + 8 * q);
        const uint32_t pw[2] = {prior.x, prior.y};
        uint32_t packed[2];
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const int e = 4 * q + r;
          float v0 = ((float)acc[i][j][e] * ws[e]) * as[i];
          float v1 = ((float)acc[i][j][e + 1] * ws[e + 1]) * as[i];
          if (EPI == kEpiBias) {
            v0 = v0 + extra[e];
            v1 = v1 + extra[e + 1];
          }
          bf16_round2(v0, v1);
          if (EPI == kEpiResid) {  // x = bf16(x + bf16(gate * bf16(v)))
            float g0 = v0 * extra[e], g1 = v1 * extra[e + 1];
            bf16_round2(g0, g1);
            const uint32_t w = pw[r >> 1];
            packed[r >> 1] = bf16_pack2(__uint_as_float(w << 16) + g0,
                                        __uint_as_float(w & 0xffff0000u) + g1);
          } else {
            packed[r >> 1] = f16_pack2(v0, v1);
          }
        }
        *reinterpret_cast<uint2 *>(out + 8 * q) = make_uint2(packed[0], packed[1]);
      }
    }
  }
}

// Epilogue through LDS (every output but split-K's int32 slices, which also go through
// it: 4-byte elements). The
// f32 arithmetic up to the stored value's rounding runs on the accumulator layout,
// as in store_tile; the packed 16-bit values then go to this wave's LDS region, one
// 32-row block at a time, and come back as 16-byte runs of eight consecutive output
// columns of one row, so every global store writes whole row segments (a store
// instruction covers 64 x 16 bytes) instead of 32 rows x 16 bytes. The residual's
// read-modify-write of x happens on that row layout, with the same f32 operations:
// the staged value is bf16(v); x = bf16(x + bf16(gate * v)).
// `region` holds 32 rows of kPitch bytes (the output columns plus 16 bytes, which
// spreads the rows' 8-byte writes over the banks).
// Per-tile epilogue operands, staged into LDS after the K loop's stages by one wave's
// transfers at the start of the tile (so their latency hides behind the K loop instead
// of stalling the epilogue): the BN channel scales, then BN per-channel extras (the f16
// bias, or the residual's f32 gate), then the BM row scales (ghost rows repeat the last).
template <int BM, int BN>
struct EpiOperands {
  static constexpr int kWs = 0, kExtra = BN * 4, kAs = BN * 8;
  static constexpr int kBytes = BN * 8 + BM * 4;
};

// The epilogue's per-wave LDS regions (32 rows of the wave's output columns plus 16
// bytes per row; 16-bit outputs). When a wave leaves the K loop, every stage but the
// last one read is free (the last barrier of the loop came after the reads of the
// others, and no transfer targets them any more), so the regions go in such a stage,
// and those that do not fit in it in an overflow area after the epilogue operands:
// each wave then starts its epilogue without waiting for the others at a barrier
// (the two waves of a SIMD leave the loop about a thousand cycles apart).
template <int BM, int BN, int WM, int WN, int BK, int STAGES, int KG>
struct EpiStaging {
  static constexpr int kWaves = WM * WN, kFN = BN / WN / 32, kStage = (BM + BN) * BK;
  static constexpr int kRegion = 32 * (32 * kFN * 2 + 16);
  static constexpr int kPerStage = kStage / kRegion < kWaves ? kStage / kRegion : kWaves;
  static constexpr int kOverflow = KG == 1 ? (kWaves - kPerStage) * kRegion : 0;
};

template <int EPI, int BM, int BN>
__device__ __forceinline__ void stage_epi_operands(const GemmArgs &g, int m0, int n0, int lane,
                                                   uint32_t lds) {
  using E = EpiOperands<BM, BN>;
  static_assert((BN * 4 <= 1024 && BM % 64 == 0) || BM < 64, "one transfer per column operand");
  if (EPI == kEpiAcc) return;
  if (lane < BN / 4) dma16(lds + E::kWs, reinterpret_cast<const int8_t *>(g.w_scale), (uint32_t)(n0 * 4 + lane * 16));
  if (EPI == kEpiBias && lane < BN / 8)
    dma16(lds + E::kExtra, reinterpret_cast<const int8_t *>(g.bias), (uint32_t)(n0 * 2 + lane * 16));
  if (EPI == kEpiResid && lane < BN / 4)
    dma16(lds + E::kExtra, reinterpret_cast<const int8_t *>(g.gate), (uint32_t)(n0 * 4 + lane * 16));
#pragma unroll
  for (int r = 0; r < BM; r += 64) {
    const int m = min(m0 + r + lane, g.m - 1);
    if (BM >= 64 || lane < BM) dma4(lds + E::kAs + r * 4, g.a_scale, (uint32_t)(m * 4));
  }
}

// Epilogue through LDS (every output but split-K's int32 slices, which also go through
// it: 4-byte elements). The
// f32 arithmetic up to the stored value's rounding runs on the accumulator layout,
// as in store_tile; the packed 16-bit values then go to this wave's LDS region, one
// 32-row block at a time, and come back as 16-byte runs of eight consecutive output
// columns of one row, so every global store writes whole row segments (a store
// instruction covers 64 x 16 bytes) instead of 32 rows x 16 bytes. The residual's
// read-modify-write of x happens on that row layout, with the same f32 operations:
// the staged value is bf16(v); x = bf16(x + bf16(gate * v)).
// `region` holds 32 rows of kPitch bytes (the output columns plus 16 bytes, which
// spreads the rows' 8-byte writes over the banks). `ops` is the tile's staged
// epilogue operands (EpiOperands), `m_off`/`n_off` this wave's offsets in the tile.
// The block's LDS reads (and the residual's reads of x) are all issued before the
// first store, so the block waits one round trip for them, not one per row run.
template <int EPI, int FM, int FN, int BM, int BN>
__device__ __forceinline__ void store_tile_lds(const GemmArgs &g, int split, v16i (&acc)[FM][FN], int m0,
                                               int n0, int m_off, int n_off, int fr, int kh, int lane,
                                               uint8_t *region, const uint8_t *ops) {
  using E = EpiOperands<BM, BN>;
  constexpr int kCols = EPI == kEpiSwiglu ? 16 * FN : 32 * FN;  // output columns
  constexpr int kElem = EPI == kEpiAcc ? 4 : 2;                  // output bytes
  constexpr int kPitch = kCols * kElem + 16;
  constexpr int kChunks = kCols * kElem / 16;  // 16-byte runs per row
  constexpr int kReads = (32 * kChunks + 63) / 64;
  const int m_base = m0 + m_off, n_base = n0 + n_off;
  const int out_base = EPI == kEpiSwiglu ? n_base / 2 : n_base;
  const float *ws_lds = reinterpret_cast<const float *>(ops + E::kWs) + n_off;
  const float *as_lds = reinterpret_cast<const float *>(ops + E::kAs) + m_off;
  // Per-channel vectors of this lane's channels: n = n_base + 32j + 8q + 4kh + r
  // (SwiGLU: registers 8-15 are the up channels, 16 further on). Read once for all row
  // blocks where the registers allow (the 256x256 tiles' SwiGLU and bias epilogues
  // would spill: they read them per block).
  constexpr bool kHoist = EPI != kEpiAcc && (FN <= 2 || EPI == kEpiPlain || EPI == kEpiResid);
  auto channel_vectors = [&](int j, float *ws, float *extra) {
    const int nb = j * 32 + kh * 4;  // within the wave's columns
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ch = (EPI == kEpiSwiglu && q >= 2) ? nb + 16 + 8 * (q - 2) : nb + 8 * q;
      const float4 v = *reinterpret_cast<const float4 *>(ws_lds + ch);
      ws[4 * q] = v.x; ws[4 * q + 1] = v.y; ws[4 * q + 2] = v.z; ws[4 * q + 3] = v.w;
      if (EPI == kEpiBias) {
        const uint2 b = *reinterpret_cast<const uint2 *>(ops + E::kExtra + 2 * (n_off + ch));
        extra[4 * q] = f16_value(b.x & 0xffffu); extra[4 * q + 1] = f16_value(b.x >> 16);
        extra[4 * q + 2] = f16_value(b.y & 0xffffu); extra[4 * q + 3] = f16_value(b.y >> 16);
      }
    }
  };
  float wsv[kHoist ? FN : 1][16], exv[kHoist && EPI == kEpiBias ? FN : 1][16];
  if constexpr (kHoist) {
#pragma unroll
    for (int j = 0; j < FN; ++j) channel_vectors(j, wsv[j], exv[EPI == kEpiBias ? j : 0]);
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const float as = EPI == kEpiAcc ? 1.0f : as_lds[i * 32 + fr];
    uint8_t *row = region + fr * kPitch;
    float sw_g[EPI == kEpiSwiglu ? FN * 8 : 2], sw_u[EPI == kEpiSwiglu ? FN * 8 : 2];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if (EPI == kEpiAcc) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<v4i *>(row + 4 * (j * 32 + 8 * q + 4 * kh)) =
              v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        continue;
      }
      float ws_b[kHoist ? 1 : 16], extra_b[kHoist ? 1 : 16];
      if constexpr (!kHoist) channel_vectors(j, ws_b, extra_b);
      const float *ws = kHoist ? wsv[j] : ws_b;
      const float *extra = kHoist ? exv[EPI == kEpiBias ? j : 0] : extra_b;
      if (EPI == kEpiSwiglu) {
        // registers 0-7: gate channels 8q+4kh+r (q<2), 8-15: the matching ups; the
        // products of the block's FN x 8 pairs are formed together (swiglu_products)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float g0 = ((float)acc[i][j][e] * ws[e]) * as;
          float g1 = ((float)acc[i][j][e + 1] * ws[e + 1]) * as;
          float u0 = ((float)acc[i][j][8 + e] * ws[8 + e]) * as;
          float u1 = ((float)acc[i][j][8 + e + 1] * ws[8 + e + 1]) * as;
          bf16_round2(g0, g1);
          bf16_round2(u0, u1);
          sw_g[j * 8 + e] = g0;
          sw_g[j * 8 + e + 1] = g1;
          sw_u[j * 8 + e] = u0;
          sw_u[j * 8 + e + 1] = u1;
        }
        continue;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t packed[2];
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const int e = 4 * q + r;
          float v0 = ((float)acc[i][j][e] * ws[e]) * as;
          float v1 = ((float)acc[i][j][e + 1] * ws[e + 1]) * as;
          if (EPI == kEpiBias) {
            v0 = v0 + extra[e];
            v1 = v1 + extra[e + 1];
          }
          if (EPI == kEpiResid) {
            packed[r >> 1] = bf16_pack2(v0, v1);
          } else {
            bf16_round2(v0, v1);
            packed[r >> 1] = f16_pack2(v0, v1);
          }
        }
        *reinterpret_cast<uint2 *>(row + 2 * (j * 32 + 8 * q + 4 * kh)) = make_uint2(packed[0], packed[1]);
      }
    }
    if constexpr (EPI == kEpiSwiglu) {
      swiglu_products(sw_g, sw_u);
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          *reinterpret_cast<uint2 *>(row + 2 * (j * 16 + 8 * q + 4 * kh)) =
              make_uint2(f16_pack2(sw_g[j * 8 + 4 * q], sw_g[j * 8 + 4 * q + 1]),
                         f16_pack2(sw_g[j * 8 + 4 * q + 2], sw_g[j * 8 + 4 * q + 3]));
    }
    // This wave's own LDS writes, read back in row order (LDS serves one wave in order):
    // first every read of the block, then the stores.
    v4u_t vals[kReads];
#pragma unroll
    for (int s = 0; s < kReads; ++s) {
      const int idx = s * 64 + lane;
      const int r = min(idx / kChunks, 31), c = idx - (idx / kChunks) * kChunks;
      vals[s] = *reinterpret_cast<const v4u_t *>(region + r * kPitch + 16 * c);
    }
    v4u_t prior[EPI == kEpiResid ? kReads : 1];
    if (EPI == kEpiResid) {
#pragma unroll
      for (int s = 0; s < kReads; ++s) {
        const int idx = s * 64 + lane;
        const int r = idx / kChunks, c = idx - r * kChunks;
        const int tok = min(m_base + i * 32 + min(r, 31), g.m - 1);
        prior[s] = *reinterpret_cast<const v4u_t *>(static_cast<const uint16_t *>(g.c) + (int64_t)tok * g.ldc +
                                                    out_base + 8 * c);
      }
    }
#pragma unroll
    for (int s = 0; s < kReads; ++s) {
      const int idx = s * 64 + lane;
      const int r = idx / kChunks, c = idx - r * kChunks;
      const int tok = m_base + i * 32 + r;
      if (r >= 32 || tok >= g.m) continue;
      v4u_t v = vals[s];
      if (EPI == kEpiAcc) {
        const int64_t at = (int64_t)tok * g.ldc + n_base + 4 * c;
        if (g.k_split_steps > 0) {
          // Split-K partial sums are written through to memory (sc1): the kernel's end
          // then has no dirty L2 lines of them to write back before the reduction kernel
          // can start (measured: 3.0 -> 1.3 us between the two at 16 MB of partials).
          // The host keeps a slice below 2 GiB, so the 32-bit buffer offset holds it.
          int32_t *slice = static_cast<int32_t *>(g.c) + (int64_t)split * g.split_stride;
          const __amdgpu_buffer_rsrc_t rsrc =
              __builtin_amdgcn_make_buffer_rsrc(slice, (short)0, 0x7fffffff, kBufferWord3);
          __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, (int)(at * 4), 0, kCachePolicySc1);
        } else {
          *reinterpret_cast<v4u_t *>(static_cast<int32_t *>(g.c) + at) = v;
        }
        continue;
      }
      uint16_t *out = static_cast<uint16_t *>(g.c) + (int64_t)tok * g.ldc + out_base + 8 * c;
      if (EPI == kEpiResid) {
        const float *gate = reinterpret_cast<const float *>(ops + E::kExtra) + n_off + 8 * c;
        const float4 g0 = *reinterpret_cast<const float4 *>(gate);
        const float4 g1 = *reinterpret_cast<const float4 *>(gate + 4);
        const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          float a0 = __uint_as_float(v[w] << 16) * gv[2 * w];
          float a1 = __uint_as_float(v[w] & 0xffff0000u) * gv[2 * w + 1];
          bf16_round2(a0, a1);
          v[w] = bf16_pack2(__uint_as_float(prior[s][w] << 16) + a0,
                            __uint_as_float(prior[s][w] & 0xffff0000u) + a1);
        }
      }
      *reinterpret_cast<v4u_t *>(out) = v;
    }
  }
}

// One output tile (workgroup number `bid` of the tile order) through the K loop and
// the epilogue: the body of gemm_kernel, callable from a persistent kernel. `smem` is
// the workgroup's dynamic LDS.
//
// KG > 1 puts KG groups of WM x WN waves on the tile, group k taking the k-th part of
// every K step's 32-byte slices; after the K loop the other groups' sums are added to
// group 0's through LDS (integer addition, exact) and group 0 runs the epilogue. On a
// small tile (64x64 with one workgroup per CU) that gives each SIMD a second wave, so
// the MFMAs of one overlap the transfer issue of the other.
//
// kBackward: the workgroups of odd rounds (one workgroup per CU, 32 CUs per XCD) step
// through their K steps last to first, so they start on what the XCD's L2 still holds
// of the previous round's last steps. The int32 sums do not depend on the order.
template <int BM, int BN, int WM, int WN, int BK, int STAGES, int EPI, int KG = 1, bool kBackward = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, int bid, uint8_t *smem) {
  constexpr int kCw = WM * WN;      // waves of one K group
  constexpr int kWaves = kCw * KG;  // waves of the workgroup
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave sub-tile
  constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 blocks per wave
  constexpr int kCpr = BK / 16;                // 16-byte chunks per staged row
  constexpr int kRowsPerKb = 1024 / BK;        // rows one transfer instruction fills
  constexpr int kAIns = BM * BK / 1024 / kWaves;  // transfers per wave per stage
  constexpr int kBIns = BN * BK / 1024 / kWaves;
  constexpr int kStage = (BM + BN) * BK;
  constexpr int kIns = kAIns + kBIns;
  static_assert(kAIns * kWaves * 1024 == BM * BK && kBIns * kWaves * 1024 == BN * BK, "staging");
  static_assert(BK % 32 == 0 && STAGES >= 2 && kWaves % 2 == 0, "pipeline");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tm, tn, split = 0;
  if (g.k_split_steps > 0)
    split_tile_of(bid, blockIdx.y, gridDim.x, gridDim.y, (g.m + BM - 1) / BM, tm, tn, split);
  else
    tile_of(bid, (g.m + BM - 1) / BM, g.n / BN, g.m_group, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // Transfers. The stage's A rows are 1 KiB blocks, block b = v*kAIns + i for "virtual
  // wave" v < kWaves (then likewise B): rows b*kRowsPerKb + lane/kCpr, physical chunk
  // lane%kCpr, which holds logical K chunk (lane%kCpr) ^ key(row). Ghost rows past m read
  // row m-1; their results are never stored. The lower half of the waves (one per SIMD)
  // issue every transfer, for virtual waves w and w + kWaves/2: a transfer instruction
  // holds up the issuing wave's next instructions for tens of cycles, and with the
  // transfers on one wave of each SIMD the other wave keeps the MFMA pipe fed meanwhile
  // (north star 159 -> 147 us against every wave issuing its own eighth).
  // Four-wave tiles (one workgroup per CU pair of SIMDs or less, the mid-M shapes) keep
  // every wave issuing its own share: there the transfers would crowd two SIMDs.
  constexpr bool kSplitRoles = kWaves == 8;
  constexpr int kHalf = kSplitRoles ? kWaves / 2 : kWaves;
  constexpr int kPer = kSplitRoles ? 2 : 1;  // virtual waves per producer
  const bool producer = wave < kHalf;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  uint32_t a_off[kPer * kAIns], b_off[kPer * kBIns];
  // This workgroup's K steps (all of K, or its split's share).
  int kt_count = g.k / BK, kt_first = 0;
  if (g.k_split_steps > 0) {
    kt_first = split * g.k_split_steps;
    kt_count = min(g.k_split_steps, kt_count - kt_first);
  }
  const uint32_t k_first = (uint32_t)(kt_first * BK);
  const int vw0 = producer ? wave : wave - kHalf;  // first virtual wave of this wave
#pragma unroll
  for (int j = 0; j < kPer; ++j)
#pragma unroll
    for (int i = 0; i < kAIns; ++i) {
      const int r = ((vw0 + j * kHalf) * kAIns + i) * kRowsPerKb + lane / kCpr;
      const int c = (lane % kCpr) ^ swz_key<BK>(r);
      a_off[j * kAIns + i] = (uint32_t)min(m0 + r, g.m - 1) * (uint32_t)g.lda + c * 16 + k_first;
    }
#pragma unroll
  for (int j = 0; j < kPer; ++j)
#pragma unroll
    for (int i = 0; i < kBIns; ++i) {
      const int r = ((vw0 + j * kHalf) * kBIns + i) * kRowsPerKb + lane / kCpr;
      const int c = (lane % kCpr) ^ swz_key<BK>(r);
      b_off[j * kBIns + i] = (uint32_t)(n0 + r) * (uint32_t)g.lda + c * 16 + k_first;
    }
  const uint32_t a_lds = lds0 + vw0 * kAIns * 1024;
  const uint32_t b_lds = lds0 + BM * BK + vw0 * kBIns * 1024;

  const bool backward = kBackward && (((bid / kXcds) / kCusPerXcd) & 1);
  auto issue = [&](int kt) {
    if (!producer) return;
    const int step = backward ? kt_count - 1 - kt : kt;
    const uint32_t so = (uint32_t)((kt % STAGES) * kStage), ko = (uint32_t)(step * BK);
#pragma unroll
    for (int j = 0; j < kPer; ++j)
#pragma unroll
      for (int i = 0; i < kAIns; ++i)
        dma16(a_lds + so + (j * kHalf * kAIns + i) * 1024, g.a, a_off[j * kAIns + i] + ko);
#pragma unroll
    for (int j = 0; j < kPer; ++j)
#pragma unroll
      for (int i = 0; i < kBIns; ++i)
        dma16(b_lds + so + (j * kHalf * kBIns + i) * 1024, g.w, b_off[j * kBIns + i] + ko);
  };
  // The epilogue's operands first: a transfer that is older than every stage's is done
  // once any wait for a stage is.
  const uint32_t ops_lds = lds0 + STAGES * kStage;
  if (wave == 0) stage_epi_operands<EPI, BM, BN>(g, m0, n0, lane, ops_lds);
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    if (s < kt_count) issue(s);

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  const int kg = wave / kCw, cw = wave - kg * kCw;
  const int wm = cw / WN, wn = cw % WN;
  const int fr = lane & 31, kh = lane >> 5;
  // Per-lane LDS byte offsets of this wave's fragment rows (chunk added per K slice;
  // a lane's fragment rows differ by multiples of 32 and share the swizzle key).
  int a_row_off[FM], b_row_off[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) a_row_off[i] = (wm * WTM + i * 32 + fr) * BK;
#pragma unroll
  for (int j = 0; j < FN; ++j) b_row_off[j] = BM * BK + (wn * WTN + j * 32 + fr) * BK;
  const int rsw = swz_key<BK>(fr);

  // Software pipeline. Fragments of the next 32-byte K slice are read while the
  // current slice's MFMAs issue; the next slice of the last slice of a step is the
  // first slice of the next stage. Before reading it, during that last slice, each
  // wave waits for its own transfers of the next stage, drains its LDS reads of the
  // current stage, and meets the others at the barrier: then every wave's transfers
  // for the next stage have landed and nobody reads the current stage any more, so
  // the transfer for stage kt+STAGES can refill it. Barrier and first reads hide
  // behind the last slice's MFMAs.
  constexpr int NS = BK / 32 / KG;  // slices of each K step per K group
  static_assert(NS % 2 == 0 && NS * KG * 32 == BK, "slice parity must repeat per step");
  const int s0 = kg * NS;  // this group's first slice of a step
  v4i af[2][FM], bf[2][FN];
  // A producer's transfers per stage: kPer kIns; the others have none outstanding.
  if (kt_count < STAGES) wait_vmcnt<0>();
  else if (producer) wait_vmcnt<(STAGES - 1) * kPer * kIns>();
  __builtin_amdgcn_s_barrier();
  read_frags<FM, FN>(af[0], bf[0], smem, a_row_off, b_row_off, ((2 * s0 + kh) ^ rsw) << 4);

  for (int kt = 0; kt < kt_count; ++kt) {
    const uint8_t *stage = smem + (kt % STAGES) * kStage;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int cur = s & 1;
      if (s + 1 < NS) {
        read_frags<FM, FN>(af[cur ^ 1], bf[cur ^ 1], stage, a_row_off, b_row_off,
                           ((2 * (s0 + s + 1) + kh) ^ rsw) << 4);
      } else {
        // lgkmcnt(0), through the builtin so that the compiler's own wait insertion
        // sees it on every path into the last slice (else it waits there for the next
        // stage's first fragment reads before the slice's first MFMAs).
        __builtin_amdgcn_s_waitcnt(0xc07f);
      }
      if (s + 1 == NS && kt + 1 < kt_count) {
        if (kt + STAGES - 1 < kt_count)
          wait_vmcnt<(STAGES - 2) * kPer * kIns>();
        else
          wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (kt + STAGES < kt_count) issue(kt + STAGES);
        read_frags<FM, FN>(af[cur ^ 1], bf[cur ^ 1], smem + ((kt + 1) % STAGES) * kStage,
                           a_row_off, b_row_off, ((2 * s0 + kh) ^ rsw) << 4);
      }
      if (s + 1 < NS) {
        // The next slice's fragment reads go one between each of the first MFMAs, so
        // the LDS requests spread over the MFMA issue instead of queueing in a burst.
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[cur][j], af[cur][i], acc[i][j], 0, 0, 0);
        constexpr int kMfma = FM * FN, kReads = FM + FN;
        constexpr int kPairs = kMfma < kReads ? kMfma : kReads;
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPairs, 0);
        if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
        __builtin_amdgcn_sched_barrier(0);
        continue;
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[cur][j], af[cur][i], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // The epilogue's LDS staging region of this wave (see EpiStaging).
  constexpr int kRegion =
      32 * ((EPI == kEpiSwiglu ? 16 * FN : 32 * FN) * (EPI == kEpiAcc ? 4 : 2) + 16);
  if constexpr (KG > 1) {
    // Groups 1.. leave their sums in LDS after group 0's epilogue regions; group 0
    // adds them. 16-byte pieces, lane-consecutive: no bank conflicts.
    constexpr int kSum = kCw * FM * FN * 64 * 64;  // bytes of one group's sums
    static_assert(kRegion * kCw + (KG - 1) * kSum <= STAGES * kStage, "K-group LDS");
    __syncthreads();
    if (kg > 0) {
      uint8_t *sums = smem + kRegion * kCw + (kg - 1) * kSum + cw * FM * FN * 64 * 64;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<v4i *>(sums + (((i * FN + j) * 4 + q) * 64 + lane) * 16) =
                v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int k = 1; k < KG; ++k) {
      const uint8_t *sums = smem + kRegion * kCw + (k - 1) * kSum + cw * FM * FN * 64 * 64;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const v4i v = *reinterpret_cast<const v4i *>(sums + (((i * FN + j) * 4 + q) * 64 + lane) * 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
          }
    }
    store_tile_lds<EPI, FM, FN, BM, BN>(g, split, acc, m0, n0, wm * WTM, wn * WTN, fr, kh, lane,
                                        smem + cw * kRegion, smem + STAGES * kStage);
  } else if constexpr ((kWaves - (kStage / kRegion < kWaves ? kStage / kRegion : kWaves)) * kRegion <=
                       EpiStaging<BM, BN, WM, WN, BK, STAGES, KG>::kOverflow) {
    constexpr int kPer = kStage / kRegion < kWaves ? kStage / kRegion : kWaves;
    const int free_stage = kt_count >= 2 ? (kt_count - 2) % STAGES : 1;
    uint8_t *region = wave < kPer ? smem + free_stage * kStage + wave * kRegion
                                  : smem + STAGES * kStage + EpiOperands<BM, BN>::kBytes + (wave - kPer) * kRegion;
    store_tile_lds<EPI, FM, FN, BM, BN>(g, split, acc, m0, n0, wm * WTM, wn * WTN, fr, kh, lane, region,
                                        smem + STAGES * kStage);
  } else if constexpr (kRegion * kWaves <= STAGES * kStage) {
    __syncthreads();
    store_tile_lds<EPI, FM, FN, BM, BN>(g, split, acc, m0, n0, wm * WTM, wn * WTN, fr, kh, lane,
                                        smem + wave * kRegion, smem + STAGES * kStage);
  } else {  // int32 output of the 256x256 tile: 135 KiB would not fit; direct stores
    store_tile<EPI, FM, FN>(g, split, acc, m0 + wm * WTM, n0 + wn * WTN, fr, kh);
  }
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES, int EPI, int KG = 1>
__global__ __launch_bounds__(WM *WN *KG * 64) void gemm_kernel(GemmArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  gemm_tile<BM, BN, WM, WN, BK, STAGES, EPI, KG>(g, blockIdx.x, smem);
}

// The same tile with odd rounds stepping through K backwards (gemm_tile's kBackward).
template <int BM, int BN, int WM, int WN, int BK, int STAGES, int EPI>
__global__ __launch_bounds__(WM *WN * 64) void gemm_kernel_backward(GemmArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  gemm_tile<BM, BN, WM, WN, BK, STAGES, EPI, 1, true>(g, blockIdx.x, smem);
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES, int KG = 1>
struct TileConfig {
  static constexpr int kThreads = WM * WN * KG * 64;
  static constexpr size_t kLds = (size_t)STAGES * (BM + BN) * BK + EpiOperands<BM, BN>::kBytes +
                                 EpiStaging<BM, BN, WM, WN, BK, STAGES, KG>::kOverflow;
};

template <int BM, int BN, int WM, int WN, int BK, int STAGES, int KG = 1>
hipError_t launch_tile(int epi, hipStream_t stream, const GemmArgs &a) {
  using T = TileConfig<BM, BN, WM, WN, BK, STAGES, KG>;
  const int tiles = ((a.m + BM - 1) / BM) * (a.n / BN);
  const int k_steps = a.k / BK;
  const int splits = a.k_split_steps > 0 ? (k_steps + a.k_split_steps - 1) / a.k_split_steps : 1;
  dim3 grid(tiles, splits), block(T::kThreads);
  switch (epi) {
    case kEpiPlain:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiPlain, KG>), grid, block, T::kLds, stream, a);
      break;
    case kEpiResid:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiResid, KG>), grid, block, T::kLds, stream, a);
      break;
    case kEpiSwiglu:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiSwiglu, KG>), grid, block, T::kLds, stream, a);
      break;
    case kEpiBias:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiBias, KG>), grid, block, T::kLds, stream, a);
      break;
    default:
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiAcc, KG>), grid, block, T::kLds, stream, a);
      break;
  }
  return hipGetLastError();
}

// The backward-K form of a wide tile (plain, residual, SwiGLU and bias epilogues).
template <int BM, int BN, int WM, int WN, int BK, int STAGES>
hipError_t launch_tile_backward(int epi, hipStream_t stream, const GemmArgs &a) {
  using T = TileConfig<BM, BN, WM, WN, BK, STAGES>;
  const int tiles = ((a.m + BM - 1) / BM) * (a.n / BN);
  dim3 grid(tiles), block(T::kThreads);
  switch (epi) {
    case kEpiPlain:
      hipLaunchKernelGGL((gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiPlain>), grid, block, T::kLds, stream, a);
      break;
    case kEpiResid:
      hipLaunchKernelGGL((gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiResid>), grid, block, T::kLds, stream, a);
      break;
    case kEpiSwiglu:
      hipLaunchKernelGGL((gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiSwiglu>), grid, block, T::kLds, stream, a);
      break;
    case kEpiBias:
      hipLaunchKernelGGL((gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiBias>), grid, block, T::kLds, stream, a);
      break;
    default:
      return launch_tile<BM, BN, WM, WN, BK, STAGES>(epi, stream, a);
  }
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES>
hipError_t set_lds_tile_backward() {
  using T = TileConfig<BM, BN, WM, WN, BK, STAGES>;
  const void *fns[4] = {reinterpret_cast<const void *>(gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiPlain>),
                        reinterpret_cast<const void *>(gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiResid>),
                        reinterpret_cast<const void *>(gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiSwiglu>),
                        reinterpret_cast<const void *>(gemm_kernel_backward<BM, BN, WM, WN, BK, STAGES, kEpiBias>)};
  for (const void *f : fns) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::kLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES, int KG = 1>
hipError_t set_lds_tile() {
  using T = TileConfig<BM, BN, WM, WN, BK, STAGES, KG>;
  const void *fns[5] = {reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiPlain, KG>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiResid, KG>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiSwiglu, KG>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiBias, KG>),
                        reinterpret_cast<const void *>(gemm_kernel<BM, BN, WM, WN, BK, STAGES, kEpiAcc, KG>)};
  for (const void *f : fns) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::kLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

inline GemmArgs args_of(const GemmLaunch &l, int epilogue) {
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
  a.ldc = (int)(epilogue == kEpiSwiglu ? l.n / 2 : l.n);
  return a;
}

}  // namespace gemm

#ifndef K2W8_GEMM_NO_ENTRY
// The 256-row tiles: eight waves, 4 (along M) x 2 (along N), 128-byte K steps, two
// stages.
constexpr int kBigWm = 4, kBigWn = 2, kBigBk = 128, kBigStages = 2;
constexpr int kMidWm = 4, kMidWn = 2;
// Stages of the 64x64 tiles: four (64 KiB, two workgroups per CU) keep three K steps
// in flight, which the short per-tile work of the mid-M shapes needs (QKV at M=256:
// 16.1 -> 9.7 us). The 128x128 tiles keep two: more would cost them occupancy.
constexpr int kS64Stages = 4, kS128Stages = 2;
// Split-K slices: 128x128 tiles of eight waves (2 x 4, each 64x32), whose lower four
// waves issue the transfers, with three stages (one workgroup per CU, two K steps in
// flight). Against four waves and two stages: M=256 down projection 19.8 -> 18.1 us,
// M=512 26.4 -> 25.0 us. Deeper 64x64 pipelines (six or eight stages, one workgroup
// per CU) were slower (QKV at M=256: 8.6 -> 9.1-9.4 us).
constexpr int kSplitStages = 3, kSplitWn = 4;
// The 64x64 tiles run as two K groups of four waves; the 128x64 tiles keep three
// stages.
constexpr int kS64Kg = 2, k12864Stages = 3;

int device_cus() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Token counts served by the few-token kernel (weights streamed, HBM-bound).
constexpr int64_t kSkinnyMaxTokens = 32;

hipError_t launch_splitk_reduce(int epilogue, hipStream_t stream, const int32_t *parts, int splits,
                                int64_t stride, const gemm::GemmArgs &g);

hipError_t configure_gemm_lds() {
  hipError_t e = gemm::set_lds_tile<256, 256, kBigWm, kBigWn, kBigBk, kBigStages>();
  if (e == hipSuccess) e = gemm::set_lds_tile<256, 192, 4, 2, 128, 2>();
  if (e == hipSuccess) e = gemm::set_lds_tile_backward<256, 256, kBigWm, kBigWn, kBigBk, kBigStages>();
  if (e == hipSuccess) e = gemm::set_lds_tile_backward<256, 192, 4, 2, 128, 2>();
  if (e == hipSuccess) e = gemm::set_lds_tile<256, 128, kMidWm, kMidWn, 128, 2>();
  if (e == hipSuccess) e = gemm::set_lds_tile<128, 128, 2, 2, 128, kS128Stages>();
  if (e == hipSuccess) e = gemm::set_lds_tile<64, 64, 2, 2, 128, kS64Stages, kS64Kg>();
  if (e == hipSuccess) e = gemm::set_lds_tile<128, 64, 4, 2, 128, k12864Stages>();
  if (e == hipSuccess) e = gemm::set_lds_tile<256, 128, kMidWm, kMidWn, 128, 3>();
  if (e == hipSuccess) e = gemm::set_lds_tile<128, 128, 2, kSplitWn, 128, kSplitStages>();
  if (e == hipSuccess) e = configure_skinny_lds();
  return e;
}

bool gemm_streams(int epilogue, const GemmLaunch &l, int64_t cus) {
  return l.m <= kSkinnyMaxTokens || skinny_streams(epilogue, l, cus);
}

// The few-token kernel, or the tile kernel plan_tiles picks (k2w8_gemm_plan.hpp).
hipError_t launch_gemm(int epilogue, hipStream_t stream, const GemmLaunch &l) {
  const int64_t cus = device_cus();
  if (gemm_streams(epilogue, l, cus)) return launch_skinny(epilogue, stream, l);
  gemm::GemmArgs a = gemm::args_of(l, epilogue);
  const TilePlan plan = plan_tiles(l.m, l.n, l.k, cus);
  // K2W8_GEMM_BACKWARD=1 (read on every call): the wide tiles' odd rounds step through
  // K backwards (gemm_tile's kBackward); the same bits, fewer L2 misses by the model.
  const char *bw = getenv("K2W8_GEMM_BACKWARD");
  const bool backward = bw && bw[0] == '1';
  switch (plan.tile) {
    case GemmTile::k256x192:
      if (backward) return gemm::launch_tile_backward<256, 192, 4, 2, 128, 2>(epilogue, stream, a);
      return gemm::launch_tile<256, 192, 4, 2, 128, 2>(epilogue, stream, a);
    case GemmTile::k256x256: {
      if (plan.n_big == 0 && backward)
        return gemm::launch_tile_backward<256, 256, kBigWm, kBigWn, kBigBk, kBigStages>(epilogue, stream, a);
      if (plan.n_big == 0) return gemm::launch_tile<256, 256, kBigWm, kBigWn, kBigBk, kBigStages>(epilogue, stream, a);
      gemm::GemmArgs big = a, tail = a;
      big.n = (int)plan.n_big;
      hipError_t e = backward
                         ? gemm::launch_tile_backward<256, 256, kBigWm, kBigWn, kBigBk, kBigStages>(epilogue, stream, big)
                         : gemm::launch_tile<256, 256, kBigWm, kBigWn, kBigBk, kBigStages>(epilogue, stream, big);
      if (e != hipSuccess) return e;
      tail.n = (int)(l.n - plan.n_big);
      tail.w = a.w + plan.n_big * l.lda;
      tail.w_scale = a.w_scale + plan.n_big;
      if (tail.gate) tail.gate = a.gate + plan.n_big;
      if (tail.bias) tail.bias = a.bias + plan.n_big;
      const int64_t out_col = epilogue == kEpiSwiglu ? plan.n_big / 2 : plan.n_big;
      const int64_t elem = epilogue == kEpiAcc ? 4 : 2;
      tail.c = static_cast<char *>(a.c) + out_col * elem;
      return gemm::launch_tile<128, 128, 2, 2, 128, kS128Stages>(epilogue, stream, tail);
    }
    case GemmTile::k256x128:
      return gemm::launch_tile<256, 128, kMidWm, kMidWn, 128, 2>(epilogue, stream, a);
    case GemmTile::k256x128Deep:
      return gemm::launch_tile<256, 128, kMidWm, kMidWn, 128, 3>(epilogue, stream, a);
    case GemmTile::k128x128:
      return gemm::launch_tile<128, 128, 2, 2, 128, kS128Stages>(epilogue, stream, a);
    case GemmTile::k128x64:
      return gemm::launch_tile<128, 64, 4, 2, 128, k12864Stages>(epilogue, stream, a);
    case GemmTile::k64x64:
      return gemm::launch_tile<64, 64, 2, 2, 128, kS64Stages, kS64Kg>(epilogue, stream, a);
    case GemmTile::kSplit:
      break;
  }
  const Workspace ws = l.workspace ? *l.workspace : splitk_workspace(stream);
  // A caller that passes a fixed workspace and requires it: a shape that would split K
  // but whose two slices do not fit is refused before anything is launched.
  if (l.workspace_required && splitk_refused(l.m, l.n, l.k, cus, ws.bytes)) return hipErrorInvalidValue;
  const int per = ws.ptr ? splitk_steps(l.m, l.n, l.k, cus, ws.bytes) : 0;
  if (per > 0) {
    int32_t *parts = static_cast<int32_t *>(ws.ptr);
    const int splits = (int)((l.k / 128 + per - 1) / per);
    gemm::GemmArgs p = a;
    p.c = parts;
    p.ldc = (int)l.n;
    p.k_split_steps = per;
    p.split_stride = l.m * l.n;
    hipError_t e = gemm::launch_tile<128, 128, 2, kSplitWn, 128, kSplitStages>(kEpiAcc, stream, p);
    if (e != hipSuccess) return e;
    return launch_splitk_reduce(epilogue, stream, parts, splits, l.m * l.n, a);
  }
  return gemm::launch_tile<64, 64, 2, 2, 128, kS64Stages, kS64Kg>(epilogue, stream, a);
}
#endif

}  // namespace k2w8
