// Activation prepares of the W8A8 path for gfx950. Each prepare forms a token's row
// in one of three ways: modulated RMSNorm, plain f16, or attention x sigmoid(gate).
// It then rotates the row by the group-256 regular Hadamard H4 (x) H4 (x) H4 (x) H4
// and quantises it per token to int8, with an f32 scale.
//
// Layout. A token row belongs to a team of WPT wave64s (one wave for widths up to 4096).
// Each lane holds T runs of 16 adjacent elements, in registers, from load to store.
// The 16 runs of a 256-group lie in one 16-lane DPP row. Lane i of the row holds run
// swap23(i), where swap23 exchanges bits 2 and 3. This maps the row's lane bits 0, 1,
// 3, 2 onto the element bits 4, 5, 6, 7 of the group. The loads and stores of a row
// still cover the group's bytes contiguously.
//
// Hadamard stages by stride:
//   1 and 4   in registers.
//   16        lanes xor 1 then xor 2, through quad_perm DPP.
//   64        lanes xor 8 (row_ror:8), then lanes xor 4 (ds_swizzle).
// The cross-lane steps keep the reference's operation order. With S = own + partner
// and D = partner - own from the first exchange, o = S - D(xor partner) equals
// (e0+e1)+(e2-e3), (e0+e1)-(e2-e3), (e0-e1)+(e2+e3) and (e2+e3)-(e0-e1) bit for bit
// (IEEE addition is commutative, and x - (-y) == x + y).
//
// The norm's sum of squares needs the reference's reduction order. For a single-wave
// team it is kept from the registers: lane l holds the reference's 32-lane-wave
// partials for virtual lanes 2r and 2r+1 of its runs r. For larger teams it runs as
// a separate canonical pass. The row amax is a wave max (plus LDS for multi-wave
// teams).
//
// Teams loop over tokens, and the next token's row is in flight while the current one
// computes. A block of single-wave teams stages the norm vectors (per element, not per
// token) in LDS once, as the factors the element formula multiplies by.
//
// Reference arithmetic: kernels/prepare_{norm,plain,gated}_i8.loom (each step below
// cites its lines).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>

#include "k2w8_numerics.hpp"
#include "k2w8_internal.hpp"

namespace k2w8 {

namespace {

enum PrepareKind { kNorm = 0, kPlain = 1, kGated = 2 };

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// DPP controls: quad_perm [1,0,3,2], [2,3,0,1]; row_ror by 8.
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowRor8 = 0x128;

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, true));
}

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Optional stage rounding of the plain prepare: f16(0.25 * o)
// (kernels/prepare_plain_i8.loom:120-127).
template <bool kQuarter>
__device__ __forceinline__ float stage_out(float o) {
  return kQuarter ? f16_round(o * 0.25f) : o;
}

// In-register radix-4 stage over quads (v[i], v[i+s], v[i+2s], v[i+3s]) of a run, in
// the reference's order (kernels/prepare_norm_i8.loom:194-201):
//   o0 = (e0+e1)+(e2-e3), o1 = (e0+e1)-(e2-e3), o2 = (e0-e1)+(e2+e3), o3 = (e2+e3)-(e0-e1).
template <int S, bool kQuarter>
__device__ __forceinline__ void radix4_reg(float (&v)[16]) {
#pragma unroll
  for (int block = 0; block < 16; block += 4 * S) {
#pragma unroll
    for (int c = 0; c < S; ++c) {
      const int i = block + c;
      const float e0 = v[i], e1 = v[i + S], e2 = v[i + 2 * S], e3 = v[i + 3 * S];
      const float s01 = e0 + e1, s23 = e2 + e3, d01 = e0 - e1, d23 = e2 - e3;
      v[i] = stage_out<kQuarter>(s01 + d23);
      v[i + S] = stage_out<kQuarter>(s01 - d23);
      v[i + 2 * S] = stage_out<kQuarter>(d01 + s23);
      v[i + 3 * S] = stage_out<kQuarter>(s23 - d01);
    }
  }
}

// The same stage on f16 values, for the plain prepare, whose every stage ends in
// f16(0.25 * o): the first sums e0 + e1, e0 - e1, ... read the f16 halves directly
// (v_fma_mix_f32: fma(e0, one, +-e1) is the f32 sum or difference of the widened
// values, rounded once), so no widening instruction precedes the stage. `one` is 1.0
// from a register: with a literal the compiler folds the fma into a widening and an add.
template <int S>
__device__ __forceinline__ void radix4_reg_f16(_Float16 (&v)[16], float one) {
#pragma unroll
  for (int block = 0; block < 16; block += 4 * S) {
#pragma unroll
    for (int c = 0; c < S; ++c) {
      const int i = block + c;
      const float s01 = __builtin_fmaf((float)v[i], one, (float)v[i + S]);
      const float d01 = __builtin_fmaf((float)v[i], one, -(float)v[i + S]);
      const float s23 = __builtin_fmaf((float)v[i + 2 * S], one, (float)v[i + 3 * S]);
      const float d23 = __builtin_fmaf((float)v[i + 2 * S], one, -(float)v[i + 3 * S]);
      v[i] = (_Float16)((s01 + d23) * 0.25f);
      v[i + S] = (_Float16)((s01 - d23) * 0.25f);
      v[i + 2 * S] = (_Float16)((d01 + s23) * 0.25f);
      v[i + 3 * S] = (_Float16)((s23 - d01) * 0.25f);
    }
  }
}

// Stride-16 stage: e0..e3 sit in lanes q = 0..3 of a quad (element bits 4, 5 = lane
// bits 0, 1). S = own + partner(xor 1) is s01 or s23; D = partner - own is -d01, d01,
// -d23, d23 for q = 0..3; o_q = S - D(q xor 2).
template <bool kQuarter>
__device__ __forceinline__ void radix4_quad(float (&v)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float s = dpp<kQuadXor1>(v[i]) + v[i];
    const float d = dpp<kQuadXor1>(v[i]) - v[i];
    v[i] = stage_out<kQuarter>(s - dpp<kQuadXor2>(d));
  }
}

// Stride-64 stage: element bit 6 = lane bit 3, bit 7 = lane bit 2. The first exchange
// is lanes xor 8 (row_ror:8, a DPP operand); the second, lanes xor 4, goes through
// ds_swizzle (bitmask mode: and 0x1f, xor 4), which has no DPP form on this chip.
template <bool kQuarter>
__device__ __forceinline__ void radix4_row(float (&v)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float s = dpp<kRowRor8>(v[i]) + v[i];
    const float d = dpp<kRowRor8>(v[i]) - v[i];
    const float dx = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, d), 0x101F));
    v[i] = stage_out<kQuarter>(s - dx);
  }
}

struct PrepareArgs {
  const uint16_t *h;      // norm: bf16 h; plain: f16 h; gated: f16 attn
  const uint16_t *gate;   // gated only
  const float *norm_scale, *mod_scale, *mod_shift;  // norm only
  int8_t *q;
  float *q_scale;
  int tokens, width, out_stride, gate_stride;
  float eps;
  int wpt;    // waves per token team
  int teams;  // teams per block
  float one;  // 1.0 (see radix4_reg_f16)
};

// bf16(sigmoid(g)) for every f16 bit pattern g, as bf16 bits: the gated prepare's
// gate factor (kernels/prepare_gated_i8.loom:97-101) depends on the 16 bits of the gate
// alone. Filled once per device by `sigmoid_table_kernel` from the same device
// functions the formula uses, so a lookup gives the formula's bits. A gated block
// copies it into LDS (128 KiB) and looks each gate up there.
__device__ __align__(16) uint16_t g_sigmoid_bf16[65536];
constexpr size_t kSigmoidTableBytes = sizeof(uint16_t) * 65536;
constexpr int kGatedWaves = 16;  // waves per gated block: one block per CU (the table)

[[maybe_unused]] __global__ __launch_bounds__(256) void sigmoid_table_kernel() {
  const int b = blockIdx.x * 256 + threadIdx.x;
  const float s = bf16_round1(sigmoid(f16_value((uint16_t)b)));
  g_sigmoid_bf16[b] = (uint16_t)(__float_as_uint(s) >> 16);
}

// Raw input of one lane for one token: T runs of 16 f16/bf16 (and the gate's).
template <int kKind, int T>
struct Raw {
  v4u x[T][2];
  v4u g[kKind == kGated ? T : 1][2];
};

constexpr int kMaxThreads = 1024;
constexpr int kFactorStride = 13;  // float4 slots per run of staged norm factors
constexpr int kMaxTeams = 16;  // most teams in a block (gated blocks pack up to 16)
constexpr int kMaxWpt = 16;

// Threads per block a kernel is compiled for: teams of up to 16 waves hold one or two
// runs per lane; three or four runs per lane need the register room of at most 8 waves.
template <int T>
struct Bounds {
  static constexpr int kThreads = T <= 2 ? kMaxThreads : 512;
};

// kSingle: one-wave teams (no block barriers, the norm's sum of squares from
// registers, norm factors staged in LDS). Otherwise teams of wpt waves.
// The prepare of the rows a block's teams own (block `block` of `blocks`): the body of
// prepare_kernel, callable from a fused kernel's producer phase. `factor_lds` is the
// block's dynamic LDS (norm factors or the sigmoid table).
template <int kKind, int T, bool kSingle>
__device__ __forceinline__ void prepare_rows(const PrepareArgs &args, int block, int blocks,
                                             float4 *factor_lds) {
  constexpr bool kQuarter = (kKind == kPlain);
  __shared__ float lds_part[2][kMaxTeams][8];         // norm partials (multi-wave teams)
  __shared__ float lds_amax[2][kMaxTeams][kMaxWpt];   // wave maxima (multi-wave teams)

  const int wpt = args.wpt, teams = args.teams;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int team = wave / wpt, wave_in_team = wave % wpt;
  const int width = args.width;
  const int runs = width >> 4;
  // Run held by this lane at t: wave base + 64 t + 16 (lane row) + swap23(lane in row).
  const int li = lane & 15;
  const int run0 = 64 * T * wave_in_team + 16 * (lane >> 4) +
                   ((li & 3) | ((li >> 3) & 1) << 2 | ((li >> 2) & 1) << 3);
  bool valid[T];
#pragma unroll
  for (int t = 0; t < T; ++t) valid[t] = run0 + 64 * t < runs;

  // Loads are unconditional (out-of-range rows and runs read row 0 / run 0 and are
  // not used), so no branch separates a prefetch from the waits on earlier loads:
  // the compiler's wait counting stays exact and the prefetch overlaps the compute.
  auto load = [&](Raw<kKind, T> &r, int token) {
    token = token < args.tokens ? token : 0;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int e0 = valid[t] ? (run0 + 64 * t) << 4 : 0;
      const v4u *p = reinterpret_cast<const v4u *>(args.h + (int64_t)token * width + e0);
      r.x[t][0] = p[0];
      r.x[t][1] = p[1];
      if (kKind == kGated) {
        const v4u *g = reinterpret_cast<const v4u *>(args.gate + (int64_t)token * args.gate_stride + e0);
        r.g[t][0] = g[0];
        r.g[t][1] = g[1];
      }
    }
  };

  const int stride = blocks * teams;
  int iter = 0;
  Raw<kKind, T> cur;
  int token = block * teams + team;
  load(cur, token);

  // Norm vectors (kernels/prepare_norm_i8.loom:150-158) as the per-element factors
  // ns + 1, bf16(ms + 1) and the shift. They do not depend on the token: a block of
  // one-wave teams stages them in LDS once (run r at float4 slots 13 r .. 13 r + 11:
  // the 208-byte run stride puts 16 consecutive runs on 16 distinct bank groups, so
  // the lanes' 16-byte reads do not conflict; a 192-byte stride repeats every 4 runs),
  // wider teams read them from global memory per token.
  constexpr bool kLdsFactors = (kKind == kNorm) && kSingle;
  if (kKind == kGated) {
    const uint4 *src = reinterpret_cast<const uint4 *>(g_sigmoid_bf16);
    for (int c = threadIdx.x; c < (int)(kSigmoidTableBytes / 16); c += blockDim.x)
      reinterpret_cast<uint4 *>(factor_lds)[c] = src[c];
    __syncthreads();
  }
  const uint16_t *sigmoid_lds = reinterpret_cast<const uint16_t *>(factor_lds);
  // Whether every modulation scale and shift is zero (plain RMSNorm, as in a block
  // without adaLN): then b = a * bf16(1 + 0) = a and c = b + 0 = b are identities (a is
  // already bf16; only the sign of a zero can change, which no code or scale sees),
  // and the formula runs without them.
  int modulated = 0;
  if (kLdsFactors) {
    for (int c = threadIdx.x; c < (width >> 2); c += blockDim.x) {
      const float4 a = reinterpret_cast<const float4 *>(args.norm_scale)[c];
      const float4 b = reinterpret_cast<const float4 *>(args.mod_scale)[c];
      const float4 sh = reinterpret_cast<const float4 *>(args.mod_shift)[c];
      modulated |= (b.x != 0.0f) | (b.y != 0.0f) | (b.z != 0.0f) | (b.w != 0.0f) |
                   (sh.x != 0.0f) | (sh.y != 0.0f) | (sh.z != 0.0f) | (sh.w != 0.0f);
      float m0 = b.x + 1.0f, m1 = b.y + 1.0f, m2 = b.z + 1.0f, m3 = b.w + 1.0f;
      bf16_round2(m0, m1);
      bf16_round2(m2, m3);
      const int slot = kFactorStride * (c >> 2) + (c & 3);
      factor_lds[slot] = make_float4(a.x + 1.0f, a.y + 1.0f, a.z + 1.0f, a.w + 1.0f);
      factor_lds[slot + 4] = make_float4(m0, m1, m2, m3);
      factor_lds[slot + 8] = sh;
    }
    modulated = __syncthreads_or(modulated);
  }
  auto factors = [&](int r, float (&ns1)[16], float (&ms1)[16], float (&shf)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 a, b, c;
      if (kLdsFactors) {
        a = factor_lds[kFactorStride * r + i];
        b = factor_lds[kFactorStride * r + 4 + i];
        c = factor_lds[kFactorStride * r + 8 + i];
      } else {
        a = reinterpret_cast<const float4 *>(args.norm_scale)[4 * r + i];
        b = reinterpret_cast<const float4 *>(args.mod_scale)[4 * r + i];
        c = reinterpret_cast<const float4 *>(args.mod_shift)[4 * r + i];
        a = make_float4(a.x + 1.0f, a.y + 1.0f, a.z + 1.0f, a.w + 1.0f);
        float m0 = b.x + 1.0f, m1 = b.y + 1.0f, m2 = b.z + 1.0f, m3 = b.w + 1.0f;
        bf16_round2(m0, m1);
        bf16_round2(m2, m3);
        b = make_float4(m0, m1, m2, m3);
      }
      ns1[4 * i] = a.x; ns1[4 * i + 1] = a.y; ns1[4 * i + 2] = a.z; ns1[4 * i + 3] = a.w;
      ms1[4 * i] = b.x; ms1[4 * i + 1] = b.y; ms1[4 * i + 2] = b.z; ms1[4 * i + 3] = b.w;
      shf[4 * i] = c.x; shf[4 * i + 1] = c.y; shf[4 * i + 2] = c.z; shf[4 * i + 3] = c.w;
    }
  };
  // The wait counter for global loads is in order: a load issued after the prefetch
  // of the next row would make every wait on it wait for the prefetch too. The
  // multi-wave norm reads the row again for its sum of squares, so it issues the
  // prefetch after that pass.
  constexpr bool kEarlyPrefetch = !(kKind == kNorm && !kSingle);

  // One token of the team: compute `cur` while the next token's row loads into `nxt`.
  auto step = [&](Raw<kKind, T> &cur, Raw<kKind, T> &nxt, auto mod_tag) __attribute__((always_inline)) {
    constexpr bool kMod = decltype(mod_tag)::value;
    const bool live = token < args.tokens;
    const int next = token + stride;
    if (kEarlyPrefetch) load(nxt, next);
    // Keep the prefetch ahead of the first use of `cur` (its wait).
    __builtin_amdgcn_sched_barrier(0);

    float rms_inv = 0.0f;
    if (kKind == kNorm) {
      // Sum of squares, kernels/prepare_norm_i8.loom:90-143. The reference's lane L of
      // 256 accumulates x^2 over chunks L, L+256, ... of 8 values into 8 partials, sums
      // them left to right, butterflies within its 32-lane wave, and adds the eight
      // wave partials as ((p0+p4)+(p2+p6))+((p1+p5)+(p3+p7)).
      float total;
      if (kSingle) {
        // Run r holds chunks 2r, 2r+1: virtual lanes (2r) mod 256 and +1, in chunk
        // sequence t/2. Lane bits 0, 1, 3, 2 are virtual-lane bits 1, 2, 3, 4.
        float acc[2][2][8];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[s][p][e] = 0.0f;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (!valid[t]) continue;
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const v4u w = cur.x[t][p];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t word = w[e >> 1];
              const float xf = (e & 1) ? hi_bf16(word) : lo_bf16(word);
              const float sq = xf * xf;
              acc[t & 1][p][e] = acc[t & 1][p][e] + sq;
            }
          }
        }
        float u[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          float sv[2];
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            float x = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) x = x + acc[s][p][e];
            sv[p] = x;
          }
          u[s] = sv[0] + sv[1];              // virtual stride 1
          u[s] = u[s] + dpp<kQuadXor1>(u[s]); // virtual stride 2
          u[s] = u[s] + dpp<kQuadXor2>(u[s]); // virtual stride 4
          u[s] = u[s] + dpp<kRowRor8>(u[s]);  // virtual stride 8
          u[s] = u[s] + __shfl_xor(u[s], 4);  // virtual stride 16
        }
        // Lane row r holds wave partials p_r (s = 0) and p_{r+4} (s = 1).
        const float pair = u[0] + u[1];
        const float half = pair + __shfl_xor(pair, 32);  // rows r, r^2
        total = half + __shfl_xor(half, 16);             // rows r, r^1
      } else {
        // Canonical pass over the row (an L2 re-read): team thread v' takes the
        // virtual lanes v' + 64 wpt k, which keep its position within a 32-lane wave.
        const int tt = wave_in_team * 64 + lane;
        const int chunks = width >> 3;
        const uint16_t *hr = args.h + (int64_t)(live ? token : 0) * width;
        for (int v = tt; v < 256; v += 64 * wpt) {
          float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          if (live) {
            for (int c = v; c < chunks; c += 256) {
              const v4u w = *reinterpret_cast<const v4u *>(hr + c * 8);
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float xf = (e & 1) ? hi_bf16(w[e >> 1]) : lo_bf16(w[e >> 1]);
                const float sq = xf * xf;
                acc[e] = acc[e] + sq;
              }
            }
          }
          float s = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) s = s + acc[e];
#pragma unroll
          for (int st = 1; st < 32; st <<= 1) s = s + __shfl_xor(s, st);
          if ((v & 31) == 0) lds_part[iter & 1][team][v >> 5] = s;
        }
        __syncthreads();
        const float *p = lds_part[iter & 1][team];
        const float pair0 = p[0] + p[4], pair1 = p[1] + p[5];
        const float pair2 = p[2] + p[6], pair3 = p[3] + p[7];
        total = (pair0 + pair2) + (pair1 + pair3);
      }
      if (!kEarlyPrefetch) {
        load(nxt, next);
        __builtin_amdgcn_sched_barrier(0);
      }
      const float mean = total / (float)width;
      const float mean_eps = mean + args.eps;
      rms_inv = 1.0f / __builtin_sqrtf(mean_eps);
    }

    // Form, rotate and bound each run.
    float v[T][16];
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (!valid[t]) continue;
      if (kKind == kNorm) {
        // kernels/prepare_norm_i8.loom:145-170
        float ns1[16], ms1[16], shf[16];
        factors(run0 + 64 * t, ns1, ms1, shf);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const uint32_t word = cur.x[t][i >> 3][(i >> 1) & 3];
          float n0 = lo_bf16(word) * rms_inv, n1 = hi_bf16(word) * rms_inv;
          float a0 = n0 * ns1[i], a1 = n1 * ns1[i + 1];
          bf16_round2(a0, a1);
          if (kMod) {
            float b0 = a0 * ms1[i], b1 = a1 * ms1[i + 1];
            bf16_round2(b0, b1);
            float c0 = b0 + shf[i], c1 = b1 + shf[i + 1];
            bf16_round2(c0, c1);
            a0 = c0;
            a1 = c1;
          }
          v[t][i] = a0;
          v[t][i + 1] = a1;
        }
      } else if (kKind == kPlain) {
        // kernels/prepare_plain_i8.loom:89-90; stages 1 and 4 on the f16 values.
        _Float16 hv[16];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const uint32_t word = cur.x[t][i >> 3][(i >> 1) & 3];
          hv[i] = __builtin_bit_cast(_Float16, (uint16_t)(word & 0xffffu));
          hv[i + 1] = __builtin_bit_cast(_Float16, (uint16_t)(word >> 16));
        }
        radix4_reg_f16<1>(hv, args.one);
        radix4_reg_f16<4>(hv, args.one);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[t][i] = (float)hv[i];
      } else {
        // kernels/prepare_gated_i8.loom:86-108
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const uint32_t aw = cur.x[t][i >> 3][(i >> 1) & 3];
          const uint32_t gw = cur.g[t][i >> 3][(i >> 1) & 3];
          float a0 = f16_value((uint16_t)(aw & 0xffffu)), a1 = f16_value((uint16_t)(aw >> 16));
          bf16_round2(a0, a1);
          // bf16(sigmoid(g)) from the table (the formula's bits).
          const float s0 = bf16_value(sigmoid_lds[gw & 0xffffu]);
          const float s1 = bf16_value(sigmoid_lds[gw >> 16]);
          float p0 = a0 * s0, p1 = a1 * s1;
          bf16_round2(p0, p1);
          v[t][i] = p0;
          v[t][i + 1] = p1;
        }
      }
      if (kKind != kPlain) {
        radix4_reg<1, kQuarter>(v[t]);
        radix4_reg<4, kQuarter>(v[t]);
      }
      radix4_quad<kQuarter>(v[t]);
      radix4_row<kQuarter>(v[t]);
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[t][i]));
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) amax = fmaxf(amax, __shfl_xor(amax, s));
    if (!kSingle) {
      if (lane == 0) lds_amax[iter & 1][team][wave_in_team] = amax;
      __syncthreads();
      for (int w = 0; w < wpt; ++w) amax = fmaxf(amax, lds_amax[iter & 1][team][w]);
    }

    // Scale (kernels/prepare_plain_i8.loom:294-299, kernels/prepare_norm_i8.loom:322-327).
    const float rotation_scale = kQuarter ? 16.0f : 0.0625f;
    const float row_max = amax * rotation_scale;
    const float safe = fmaxf(row_max, 1e-30f);
    const float scale = safe / 127.0f;
    const float inv = rotation_scale / scale;

    // Quantise and store 16 bytes per run (:301-340, bytes low first).
    if (live) {
      int8_t *qr = args.q + (int64_t)token * args.out_stride;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        if (!valid[t]) continue;
        v4u out;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t biased[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            // clamp(rne(x), +-127) == rne(clamp(x, +-127)) as the bounds are integers
            // (a NaN clamps to -127 either way). Adding 1.5 * 2^23 rounds to the
            // nearest even integer, left in the low mantissa bits in two's complement.
            float qv = v[t][4 * i + b] * inv;
            qv = fmaxf(qv, -127.0f);
            qv = fminf(qv, 127.0f);
            biased[b] = __float_as_uint(qv + 12582912.0f);
          }
          // Low bytes of the four words, in order (v_perm selector 0x0c gives 0).
          out[i] = __builtin_amdgcn_perm(biased[1], biased[0], 0x0c0c0400u) |
                   __builtin_amdgcn_perm(biased[3], biased[2], 0x04000c0cu);
        }
        *reinterpret_cast<v4u *>(qr + ((run0 + 64 * t) << 4)) = out;
      }
      if (wave_in_team == 0 && lane == 0) args.q_scale[token] = scale;
    }
    token = next;
    ++iter;
  };

  // Two row buffers in turn (no copy between iterations, so the prefetch never waits
  // on the row being computed). Every team of the block runs the same number of
  // steps (barriers inside).
  Raw<kKind, T> other;
  auto loop = [&](auto mod_tag) __attribute__((always_inline)) {
    for (int base = block * teams; base < args.tokens; base += 2 * stride) {
      step(cur, other, mod_tag);
      if (base + stride >= args.tokens) break;
      step(other, cur, mod_tag);
    }
  };
  if (!kLdsFactors || modulated)
    loop(std::true_type{});
  else
    loop(std::false_type{});
}

template <int kKind, int T, bool kSingle>
__global__ __launch_bounds__(Bounds<T>::kThreads) void prepare_kernel(PrepareArgs args) {
  extern __shared__ float4 factor_lds[];
  prepare_rows<kKind, T, kSingle>(args, blockIdx.x, gridDim.x, factor_lds);
}

#ifndef K2W8_PREPARE_NO_ENTRY
// Waves per CU the persistent grid aims for: enough to cover load latency while each
// team still loops over several tokens. The norm prepare's one-wave teams do better
// with fewer, longer-lived waves, whose prefetch of the next row overlaps the current
// row's compute (a round of one row per wave loads everything, then computes): with
// cold rows, M=4544 20.6 -> 19.5 us, width 4096 24.6 -> 23.3 us. The gated prepare
// loses a third at 8 (24.4 -> 35.0 us).
constexpr int kPrepareWavesPerCu = 32, kNormWavesPerCu = 8;

template <int kKind, int T, bool kSingle>
hipError_t launch_team(hipStream_t stream, const PrepareArgs &a) {
  const int threads = 64 * a.wpt * a.teams;
  const int needed = (a.tokens + a.teams - 1) / a.teams;
  const int waves = (kKind == kNorm && kSingle) ? kNormWavesPerCu
                    : kKind == kGated            ? kGatedWaves
                                                 : kPrepareWavesPerCu;
  int per_cu = waves / (a.wpt * a.teams);
  if (per_cu < 1) per_cu = 1;
  const int cap = device_cus() * per_cu;
  dim3 grid(needed < cap ? needed : cap), block(threads);
  const size_t lds = (kKind == kNorm && kSingle) ? (size_t)(a.width / 16) * kFactorStride * 16
                     : kKind == kGated            ? kSigmoidTableBytes
                                                  : 0;
  hipLaunchKernelGGL((prepare_kernel<kKind, T, kSingle>), grid, block, lds, stream, a);
  return hipGetLastError();
}


// Team shape for a row: the fewest waves (at most 16) that hold it with at most
// `max_runs` runs of 16 elements per lane; single-wave teams are packed four to a
// block and two-wave teams two to a block.
void team_shape(PrepareArgs &a, int max_runs, bool gated, int &t) {
  const int runs = a.width >> 4;
  int wpt = (runs + 64 * max_runs - 1) / (64 * max_runs);
  if (wpt > kMaxWpt) wpt = kMaxWpt;
  t = (runs + 64 * wpt - 1) / (64 * wpt);
  if (t > 2 && wpt > 8) {  // more than 8 waves of three or four runs: use two runs
    t = 2;
    wpt = (runs + 127) / 128;
  }
  a.wpt = wpt;
  a.teams = wpt == 1 ? 4 : (wpt == 2 ? 2 : 1);
  // A gated block holds the sigmoid table in LDS: one block per CU, as many teams as
  // fit 16 waves.
  if (gated) a.teams = kGatedWaves / wpt;
}

template <int kKind, bool kSingle>
hipError_t launch_t(int t, hipStream_t stream, const PrepareArgs &a) {
  switch (t) {
    case 1: return launch_team<kKind, 1, kSingle>(stream, a);
    case 2: return launch_team<kKind, 2, kSingle>(stream, a);
    case 3: return launch_team<kKind, 3, kSingle>(stream, a);
    default: return launch_team<kKind, 4, kSingle>(stream, a);
  }
}

template <int kKind>
hipError_t launch_kind(hipStream_t stream, PrepareArgs a) {
  // Runs of 16 elements per lane, at most: the norm keeps rows of up to 4096 in one
  // wave (sum of squares from registers, factors in LDS); the plain prepare takes
  // three (fewer waves per row: 9728 wide 50.5 -> 41.8 us at M=4096); the gated one
  // one (more waves per row: its sigmoid makes each element dearer).
  constexpr int kRuns = kKind == kNorm ? 4 : (kKind == kPlain ? 3 : 1);
  int t = 1;
  team_shape(a, kRuns, kKind == kGated, t);
  if (a.wpt == 1) return launch_t<kKind, true>(t, stream, a);
  return launch_t<kKind, false>(t, stream, a);
}

#endif  // K2W8_PREPARE_NO_ENTRY
}  // namespace
#ifndef K2W8_PREPARE_NO_ENTRY

hipError_t launch_prepare(int kind, hipStream_t stream, int64_t tokens, const PrepareLaunch &p) {
  PrepareArgs a;
  a.h = static_cast<const uint16_t *>(p.h);
  a.gate = static_cast<const uint16_t *>(p.gate);
  a.norm_scale = p.norm_scale;
  a.mod_scale = p.mod_scale;
  a.mod_shift = p.mod_shift;
  a.q = p.q;
  a.q_scale = p.q_scale;
  a.tokens = (int)tokens;
  a.width = (int)p.width;
  a.out_stride = (int)p.out_stride;
  a.gate_stride = (int)p.gate_stride;
  a.eps = p.eps;
  a.one = 1.0f;
  switch (kind) {
    case kNorm: return launch_kind<kNorm>(stream, a);
    case kPlain: return launch_kind<kPlain>(stream, a);
    default: return launch_kind<kGated>(stream, a);
  }
}

// The prepares use static LDS only.
hipError_t configure_prepare_lds() {
  // The gated prepare's sigmoid table (128 KiB of dynamic LDS).
  const void *fns[8] = {reinterpret_cast<const void *>(prepare_kernel<kGated, 1, true>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 2, true>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 3, true>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 4, true>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 1, false>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 2, false>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 3, false>),
                        reinterpret_cast<const void *>(prepare_kernel<kGated, 4, false>)};
  for (const void *f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSigmoidTableBytes);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// The sigmoid table of the current device, filled on its first use there: on `stream`,
// which is then synchronised, so that calls on any stream of the device find it
// complete. A stream capture cannot run it (the fill would only be recorded), so the
// first use on a device must come before any capture; k2w8_prime_launches does it.
hipError_t prepare_gated_ready(hipStream_t stream) {
  static std::mutex mu;
  constexpr int kMaxDevices = 64;
  static bool ready[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (ready[dev]) return hipSuccess;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &capture);
  if (e != hipSuccess) return e;
  if (capture != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
  hipLaunchKernelGGL(sigmoid_table_kernel, dim3(256), dim3(256), 0, stream);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e == hipSuccess) ready[dev] = true;
  return e;
}

#endif  // K2W8_PREPARE_NO_ENTRY

}  // namespace k2w8
