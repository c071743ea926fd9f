// The attention step of a block, between the fused qkvg GEMM and the gated prepare
// (src/session/mod.rs:714-755): per-head RMSNorm + rotary embedding on q and k, the
// V transpose, and fp16 grouped-query attention with an f32 online softmax.
//
//   rope_qknorm  kernels/rope_qknorm_f16.loom:1-159
//   v_transpose  kernels/native/v_transpose.loom (V [tokens][width] -> [width][capacity])
//   attention    kernels/attention_gqa_lds_f16_wmma.loom:1-380 (and its 32-query twin)
//
// rope_qknorm and v_transpose are HBM-bound elementwise passes. The attention kernel
// is MFMA-bound: a workgroup of four waves owns one key-value head and its `group`
// query heads (4 in the reference's layout: one wave per query head, 32 query tokens;
// 2: two waves per head, 64 tokens; 1: 128 tokens). Each 64-key tile of K and V^T is staged once
// in LDS and serves all four waves. A wave computes S^T = K Q^T with
// v_mfma_f32_32x32x16_f16 (keys as rows), so each lane holds one query's scores and
// the softmax needs only one cross-lane exchange (lanes l and l^32); the f16
// probabilities then feed O^T = V^T P^T straight from the accumulator registers, and
// the per-query rescale is a per-lane scalar.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k2w8_internal.hpp"
#include "k2w8_numerics.hpp"

namespace k2w8 {

namespace attn {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;

// ---------------------------------------------------------------------------------
// rope_qknorm: one 16-lane group per (token, head); lane j holds channels 8j..8j+7 of
// the head. Heads [0, q_heads) are q, then kv_heads of k, then kv_heads of v (copied).
//   ss   = sum of squares: lane partial ((x0^2+x1^2)+(x2^2+x3^2))+((x4^2+x5^2)+(x6^2+x7^2)),
//          then an xor butterfly over offsets 1, 2, 4, 8 (every lane ends with the same sum)
//   r    = 1 / sqrt(ss * (1/128) + eps)                     (correctly rounded)
//   x    = bf16((h * r) * (scale[c] + 1))
//   out  = f16(bf16(x[c] * cos[c] -/+ x[partner] * sin[c]))  (pairs 2i, 2i+1)
// ---------------------------------------------------------------------------------
struct RopeArgs {
  const uint16_t *qkv;
  const float *q_scale, *k_scale, *cos, *sin;
  uint16_t *q_out, *k_out, *v_out;
  uint32_t items;  // tokens * heads
  int heads, row_stride, q_heads, kv_heads, k_offset;
  float eps;
};

__device__ __forceinline__ float unpack_lo(uint32_t w) { return f16_value((uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float unpack_hi(uint32_t w) { return f16_value((uint16_t)(w >> 16)); }

__global__ __launch_bounds__(256) void rope_qknorm_kernel(RopeArgs r) {
  const uint32_t item = blockIdx.x * 16u + (threadIdx.x >> 4);
  const int j = threadIdx.x & 15;
  if (item >= r.items) return;  // the 16 lanes of an item leave together
  const uint32_t t = item / (uint32_t)r.heads;
  const int head = (int)(item - t * (uint32_t)r.heads);
  const bool is_q = head < r.q_heads;
  const bool is_v = head >= r.q_heads + r.kv_heads;
  const int kh = is_q ? 0 : head - r.q_heads;
  const int vh = is_v ? head - r.q_heads - r.kv_heads : 0;
  const int col = is_q ? head * 128 : (is_v ? r.k_offset + r.kv_heads * 128 + vh * 128 : r.k_offset + kh * 128);
  const v4u in = *reinterpret_cast<const v4u *>(r.qkv + (int64_t)t * r.row_stride + col + 8 * j);
  const int64_t kv_row = (int64_t)t * r.kv_heads * 128;
  if (is_v) {
    *reinterpret_cast<v4u *>(r.v_out + kv_row + vh * 128 + 8 * j) = in;
    return;
  }
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = unpack_lo(in[i]);
    x[2 * i + 1] = unpack_hi(in[i]);
  }
  float ss = ((x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3])) +
             ((x[4] * x[4] + x[5] * x[5]) + (x[6] * x[6] + x[7] * x[7]));
  ss += __shfl_xor(ss, 1, 16);
  ss += __shfl_xor(ss, 2, 16);
  ss += __shfl_xor(ss, 4, 16);
  ss += __shfl_xor(ss, 8, 16);
  const float rinv = 1.0f / __builtin_sqrtf(ss * 0.0078125f + r.eps);
  const float *scale = (is_q ? r.q_scale : r.k_scale) + 8 * j;
  const float4 s0 = *reinterpret_cast<const float4 *>(scale);
  const float4 s1 = *reinterpret_cast<const float4 *>(scale + 4);
  const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const float *cs = r.cos + (int64_t)t * 128 + 8 * j;
  const float *sn = r.sin + (int64_t)t * 128 + 8 * j;
  const float4 c0 = *reinterpret_cast<const float4 *>(cs), c1 = *reinterpret_cast<const float4 *>(cs + 4);
  const float4 n0 = *reinterpret_cast<const float4 *>(sn), n1 = *reinterpret_cast<const float4 *>(sn + 4);
  const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sv[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
  v4u o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = (x[2 * i] * rinv) * (sc[2 * i] + 1.0f);
    float b = (x[2 * i + 1] * rinv) * (sc[2 * i + 1] + 1.0f);
    bf16_round2(a, b);
    float ra = a * cv[2 * i] - b * sv[2 * i];
    float rb = b * cv[2 * i + 1] + a * sv[2 * i + 1];
    bf16_round2(ra, rb);
    o[i] = f16_pack2(ra, rb);
  }
  uint16_t *dst = is_q ? r.q_out + (int64_t)t * r.q_heads * 128 + head * 128 : r.k_out + kv_row + kh * 128;
  *reinterpret_cast<v4u *>(dst + 8 * j) = o;
}

// ---------------------------------------------------------------------------------
// v_transpose: [rows][width] f16 -> [width][capacity] f16 through a 64x64 LDS tile.
// Output columns at or past `rows` are never written (the caller's zero headroom).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void v_transpose_kernel(const uint16_t *x, uint16_t *out, int rows,
                                                          int width, int capacity) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][72];
  const int r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int row = (tid >> 3) + 32 * p, ch = (tid & 7) * 8;
    v4u v = {0u, 0u, 0u, 0u};
    if (r0 + row < rows && c0 + ch < width)
      v = *reinterpret_cast<const v4u *>(x + (int64_t)(r0 + row) * width + c0 + ch);
    *reinterpret_cast<v4u *>(&tile[row][ch]) = v;
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int ch = (tid >> 3) + 32 * p, tk = (tid & 7) * 8;
    if (c0 + ch >= width) continue;
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = tile[tk + i][ch];
    uint16_t *dst = out + (int64_t)(c0 + ch) * capacity + r0 + tk;
    if (r0 + tk + 8 <= rows) {
      v4u v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (uint32_t)e[2 * i] | ((uint32_t)e[2 * i + 1] << 16);
      *reinterpret_cast<v4u *>(dst) = v;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (r0 + tk + i < rows) dst[i] = e[i];
    }
  }
}

// ---------------------------------------------------------------------------------
// attention: grid of (query blocks of 128/group tokens) x kv_heads workgroups,
// renumbered XCD-major so that the workgroups of one key-value head share an XCD's L2.
// 256 threads: wave w computes query head kv_head*group + w % group for the 32 query
// tokens starting at the block's first + 32 * (w / group).
//
// LDS, two stages of 32 KiB, filled by global_load_lds_dwordx4 (no staging registers):
//   K tile   [64 rows][128 ch] f16, 256-byte rows; row r holds key perm(r), which swaps
//            bits 2 and 3 of r, so that a lane half's eight score registers of a 16-key
//            group are eight consecutive keys. 16-byte chunk c of row r at c ^ (r & 15).
//   V^T tile [128 ch][64 keys] f16, 128-byte rows in key order; chunk c of row r at
//            c ^ ((r >> 1) & 7).
// Two workgroups share a CU (LDS 64 KiB and at most 256 registers per lane each), so a
// SIMD interleaves one wave's softmax with another's MFMAs. The online softmax keeps a
// per-query reference point m for exp2(s - m) that moves only when a score exceeds it
// by more than kLag, so the accumulators are rarely rescaled.
// ---------------------------------------------------------------------------------
struct AttnArgs {
  const uint16_t *q, *k, *vt;
  uint16_t *out;
  int tokens, rows_out, capacity, q_stride, kv_stride, out_stride, kv_heads, q_blocks, group;
  float scale_log2;  // scale * log2(e): softmax in base 2
};

constexpr int kKeys = 64;
constexpr float kLag = 8.0f;  // how far (log2 units) a score may exceed the exponent's reference point
constexpr int kStage = 2 * 16384;

__device__ __forceinline__ int key_of_row(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
__device__ __forceinline__ int k_addr(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }
__device__ __forceinline__ int v_addr(int row, int chunk) {
  return 16384 + row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
}

__device__ __forceinline__ const void *uniform_ptr(const void *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void *>(((uint64_t)hi << 32) | lo);
}

// Lane l writes LDS bytes [lds + 16 l, +16) from global base + voff (bytes).
__device__ __forceinline__ void dma16(uint32_t lds, const void *base, uint32_t voff) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform_ptr(base)), "{m0}"(lds) : "memory");
}

// Scores are never NaN, and this file is compiled with -fno-honor-nans: the maximum
// selects v_max3_f32 without NaN-quieting copies of MFMA results. (An inline-asm
// v_max3 would hide the MFMA result read from the compiler's hazard tracking, which
// inserts the wait states a VALU read of an MFMA result needs.)
__device__ __forceinline__ float max3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

// The value lane l ^ 32 holds. v_permlane32_swap exchanges lanes 32-63 of its first
// operand with lanes 0-31 of its second: with x in both, the first result holds
// x[l - 32] in the upper half and the second x[l + 32] in the lower half.
__device__ __forceinline__ float across_halves(float x, int hf) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(hf ? r[0] : r[1]);
}

__global__ __launch_bounds__(256, 2) void attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];
  // XCD-major renumbering: consecutive workgroups land on XCDs round-robin.
  int bid = blockIdx.x;
  const int total = a.q_blocks * a.kv_heads;
  const int per_xcd = total / kXcds;
  if (bid < per_xcd * kXcds) bid = (bid % kXcds) * per_xcd + bid / kXcds;
  const int kv_head = bid / a.q_blocks;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, hf = lane >> 5;
  const int head = kv_head * a.group + wave % a.group;
  const int q0 = (bid - kv_head * a.q_blocks) * (128 / a.group) + 32 * (wave / a.group);

  // Transfers of one tile: wave w fills K rows 16w..16w+15 and V^T rows 32w..32w+31,
  // four 1 KiB instructions each; byte offsets from the tile's first key.
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  // Key row j of this lane's K transfers, the first key of its V^T transfers.
  auto k_row_of = [&](int j) { return key_of_row(16 * wave + 4 * j + (lane >> 4)); };
  auto v_key_of = [&](int j) { return ((lane & 7) ^ (((32 * wave + 8 * j + (lane >> 3)) >> 1) & 7)) * 8; };
  uint32_t k_off[4], v_off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 16 * wave + 4 * j + (lane >> 4);
    const int k_col = ((lane & 15) ^ (r & 15)) * 8;
    k_off[j] = (uint32_t)(k_row_of(j) * a.kv_stride + k_col) * 2u;
    const int vr = 32 * wave + 8 * j + (lane >> 3);
    v_off[j] = (uint32_t)(vr * a.capacity + v_key_of(j)) * 2u;
  }
  const uint16_t *k_head = a.k + kv_head * 128;
  const uint16_t *v_head = a.vt + (int64_t)kv_head * 128 * a.capacity;
  const int tiles = (a.tokens + kKeys - 1) / kKeys;
  auto issue = [&](int t, uint32_t so) __attribute__((always_inline)) {
    const int key0 = t * kKeys;
    const uint16_t *kb = k_head + (int64_t)key0 * a.kv_stride;
    const uint16_t *vb = v_head + key0;
    if (key0 + kKeys <= a.capacity) {
#pragma unroll
      for (int j = 0; j < 4; ++j) dma16(so + (4 * wave + j) * 1024, kb, k_off[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j) dma16(so + 16384 + (4 * wave + j) * 1024, vb, v_off[j]);
    } else {  // the last tile may reach past the buffers' rows: clamp (those keys are masked)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = min(key0 + k_row_of(j), a.capacity - 1) - key0;
        dma16(so + (4 * wave + j) * 1024, kb, k_off[j] + (uint32_t)((key - k_row_of(j)) * a.kv_stride) * 2u);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int first = min(key0 + v_key_of(j), a.capacity - 8) - key0;
        dma16(so + 16384 + (4 * wave + j) * 1024, vb, v_off[j] + (uint32_t)(first - v_key_of(j)) * 2u);
      }
    }
  };

  // This lane's query (column of S^T): 8 K-steps of 16 channels, 8 per lane half.
  v8h qf[8];
  {
    const int qt = min(q0 + col, a.capacity - 1);
    const uint16_t *qrow = a.q + (int64_t)qt * a.q_stride + head * 128 + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const v8h *>(qrow + 16 * ks);
    // Consume the loads here: a first use inside the tile loop would make the compiler
    // wait on the loop's later transfers (vmcnt counts both) in every iteration.
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) asm volatile("" ::"v"(qf[ks]));
  }

  v16f o[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[cb][i] = 0.0f;
  float m_run = -__builtin_inff(), l_run = 0.0f;
  const float c = a.scale_log2;
  // Per-lane LDS byte offsets within a stage of the K and V^T fragment rows.
  // Rows kb*32 + col and cb*32 + col share the swizzle of row col: the blocks are
  // constant offsets (8192 kb, 4096 cb) from the row-col addresses.
  int k_frag[8], v_frag[4];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) k_frag[ks] = k_addr(col, 2 * ks + hf);
#pragma unroll
  for (int g = 0; g < 4; ++g) v_frag[g] = v_addr(col, 2 * g + hf);

  // One tile on a stage whose offset is a compile-time constant at each call.
  auto step = [&](int t, const int stage_off) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (t + 1 < tiles) issue(t + 1, lds0 + (stage_off ^ kStage));
    const uint8_t *stage = lds + stage_off;
    const int key0 = t * kKeys;

    // S^T for 64 keys: two 32-row blocks. s[kb][i] is key
    // key0 + 32kb + 16(i/8) + 8hf + i%8.
    // The two blocks' MFMA chains alternate, so no MFMA waits on the one before it.
    v16f s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const v8h kf = *reinterpret_cast<const v8h *>(stage + kb * 8192 + k_frag[ks]);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[kb], 0, 0, 0);
      }

    // Online softmax in base 2, on raw scores scaled inside the exponent.
    if (key0 + kKeys > a.tokens) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (key0 + 32 * kb + 16 * (i >> 3) + 8 * hf + (i & 7) >= a.tokens) s[kb][i] = -__builtin_inff();
    }
    float mx[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v16f &sv = s[g >> 1];
      const int b = (g & 1) * 8;
      mx[g] = max3(max3(max3(sv[b], sv[b + 1], sv[b + 2]), sv[b + 3], sv[b + 4]),
                   max3(sv[b + 5], sv[b + 6], sv[b + 7]), sv[b]);
    }
    float m_tile = max3(max3(mx[0], mx[1], mx[2]), mx[3], mx[3]);
    m_tile = max3(m_tile, across_halves(m_tile, hf), m_tile) * c;
    // The reference point of the exponent moves only when the tile's maximum exceeds
    // it by more than kLag (base 2): weights stay below 2^kLag (f16 holds them at full
    // relative precision), and the accumulators are rescaled far less often. Any
    // reference point gives the same softmax after the final division.
    const float m_new = m_tile > m_run + kLag ? m_tile : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float part[4];
    v8h pf[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v16f &sv = s[g >> 1];
      const int b = (g & 1) * 8;
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[b + e], c, -m_new));
      part[g] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      v4u packed;
#pragma unroll
      for (int e = 0; e < 4; ++e) packed[e] = f16_pack2(p[2 * e], p[2 * e + 1]);
      pf[g] = __builtin_bit_cast(v8h, packed);
    }
    l_run = l_run * alpha + ((part[0] + part[1]) + (part[2] + part[3]));
    // Rescale only when some query's maximum moved (alpha == 1 leaves o as it is).
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[cb][i] *= alpha;
    }

    // O^T += V^T P^T over the tile's four 16-key groups (four independent chains).
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const v8h vf = *reinterpret_cast<const v8h *>(stage + cb * 4096 + v_frag[g]);
        o[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[g], o[cb], 0, 0, 0);
      }
  };

  issue(0, lds0);
  for (int t = 0; t < tiles; t += 2) {
    step(t, 0);
    if (t + 1 < tiles) step(t + 1, kStage);
  }


  // Row sums: each lane half holds the partial over its keys.
  const float inv = 1.0f / (l_run + across_halves(l_run, hf));
  const int qt = q0 + col;
  if (qt >= a.rows_out) return;
  uint16_t *orow = a.out + (int64_t)qt * a.out_stride + head * 128;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int ch = cb * 32 + 8 * g4 + 4 * hf;
      uint2 v;
      v.x = f16_pack2(o[cb][4 * g4] * inv, o[cb][4 * g4 + 1] * inv);
      v.y = f16_pack2(o[cb][4 * g4 + 2] * inv, o[cb][4 * g4 + 3] * inv);
      *reinterpret_cast<uint2 *>(orow + ch) = v;
    }
}

}  // namespace attn

hipError_t launch_rope_qknorm(hipStream_t stream, const RopeLaunch &l) {
  attn::RopeArgs r;
  r.qkv = static_cast<const uint16_t *>(l.qkv);
  r.q_scale = l.q_scale;
  r.k_scale = l.k_scale;
  r.cos = l.cos;
  r.sin = l.sin;
  r.q_out = static_cast<uint16_t *>(l.q_out);
  r.k_out = static_cast<uint16_t *>(l.k_out);
  r.v_out = static_cast<uint16_t *>(l.v_out);
  r.heads = (int)(l.q_heads + 2 * l.kv_heads);
  r.items = (uint32_t)(l.tokens * r.heads);
  r.row_stride = (int)l.row_stride;
  r.q_heads = (int)l.q_heads;
  r.kv_heads = (int)l.kv_heads;
  r.k_offset = (int)l.k_offset;
  r.eps = l.eps;
  dim3 grid((r.items + 15) / 16), block(256);
  hipLaunchKernelGGL(attn::rope_qknorm_kernel, grid, block, 0, stream, r);
  return hipGetLastError();
}

hipError_t launch_v_transpose(hipStream_t stream, int64_t rows, int64_t width, int64_t capacity,
                              const void *x, void *out) {
  dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((width + 63) / 64)), block(256);
  hipLaunchKernelGGL(attn::v_transpose_kernel, grid, block, 0, stream, static_cast<const uint16_t *>(x),
                     static_cast<uint16_t *>(out), (int)rows, (int)width, (int)capacity);
  return hipGetLastError();
}

hipError_t launch_attention(hipStream_t stream, const AttentionLaunch &l) {
  attn::AttnArgs a;
  a.q = static_cast<const uint16_t *>(l.q);
  a.k = static_cast<const uint16_t *>(l.k);
  a.vt = static_cast<const uint16_t *>(l.vt);
  a.out = static_cast<uint16_t *>(l.out);
  a.tokens = (int)l.tokens;
  a.rows_out = (int)l.rows_out;
  a.capacity = (int)l.capacity;
  a.q_stride = (int)l.q_stride;
  a.kv_stride = (int)l.kv_stride;
  a.out_stride = (int)l.out_stride;
  a.kv_heads = (int)l.kv_heads;
  a.group = (int)l.group;
  a.q_blocks = (int)((l.tokens + 128 / l.group - 1) / (128 / l.group));
  a.scale_log2 = (float)((double)l.scale * 1.4426950408889634);
  dim3 grid((unsigned)(a.q_blocks * a.kv_heads)), block(256);
  hipLaunchKernelGGL(attn::attention_kernel, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace k2w8
