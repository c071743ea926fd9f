/*
 * CPU restatement of krea2-hrx's W8A8 transformer-product path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP kernels and the
 * timed CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. It is built with -ffp-contract=off so every
 * f32 operation below rounds exactly where it is written.
 *
 * Each function cites the reference file:line whose arithmetic it restates
 * (paths under zacharydenton/krea2-hrx).
 *
 * Pinning (what independently checks each part, in tests/test_oracle.py):
 *   prepare_plain     bit-exact known-answer test of tests/quantized.rs:514-569
 *   prepare_norm      Kronecker-Hadamard tolerance test of tests/quantized.rs:385-512,
 *                     plus the sum-of-squares against an f64 sum; the in-wave
 *                     reduction order and rsqrt precision are fixed by the reference's
 *                     third-party Loom compiler, so bit parity is unpinned
 *                     (canonical order defined in ora_norm_sum_squares below)
 *   prepare_gated     Kronecker-Hadamard tolerance test; exp is this file's own
 *                     (the reference uses a compiler approximation): bit parity unpinned
 *   gemm_i32          brute-force integer dot of tests/quantized.rs:203-211
 *   epilogue_plain    exact KAT src/training/quantized.rs:220
 *   epilogue_resid    tests/quantized.rs:229-243 tolerance + closed form
 *   epilogue_swiglu   tests/quantized.rs:244-255 tolerance (exp unpinned, as above)
 *   epilogue_bias     no reference counterpart (an extension); pinned by the arithmetic:
 *                     a +-0 bias gives epilogue_plain bit for bit, a zero accumulator
 *                     gives f16(bf16(bias)), and every output is within one bf16 ulp plus
 *                     the f32 error bound of the f64 closed form acc*ws*as + bias
 *   gemm_i8           the fused CPU GEMM (the timed baseline): equal to gemm_i32 followed
 *                     by epilogue_plain, on one thread and on all
 *   f16 / bf16        numpy binary16 and torch bfloat16 over random bit patterns and
 *                     every class (zeros, subnormals, overflow boundary, infinities)
 *   rope_qknorm       tolerance test of tests/quantized.rs:85-166 against an f64 norm,
 *                     the f32 rotary sum and the exact v copy; the in-wave sum-of-squares
 *                     order and rsqrt are the Loom compiler's, so bit parity is unpinned
 *                     (canonical order in ora_head_sum_squares)
 *   v_transpose       exact: a permutation, checked against numpy's transpose
 *   attention         tests/quantized.rs:313-380 tolerance against an f64 softmax;
 *                     the reference's exp and MMA summation order belong to its compiler
 *                     and hardware: parity is a tolerance, not bits
 */
#include "w8a8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t bits_of(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}
static inline float float_of(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* src/numerics.rs:18-26: round to nearest even on the f32 bit pattern, NaN quieted. */
uint16_t ora_bf16_from_f32(float x) {
    uint32_t u = bits_of(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float ora_bf16_to_f32(uint16_t b) { return float_of((uint32_t)b << 16); }

/* Round-to-nearest-even f32 -> IEEE binary16, overflow to infinity. */
uint16_t ora_f16_from_f32(float x) {
    uint32_t u = bits_of(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t ax = u & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (ax >= 0x38800000u) {                                  /* >= 2^-14: normal */
        uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u) - 0x38000000u;
        return (uint16_t)(sign | (r >> 13));
    }
    /* subnormal: count units of 2^-24; the scaling is exact, rintf rounds to even */
    float units = fabsf(x) * 16777216.0f;
    return (uint16_t)(sign | (uint16_t)rintf(units));
}

float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return float_of(sign | 0x7f800000u | (m << 13));
    return float_of(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float bf_round(float x) { return ora_bf16_to_f32(ora_bf16_from_f32(x)); }
static inline float f16_round(float x) { return ora_f16_to_f32(ora_f16_from_f32(x)); }

/*
 * exp(x) for the sigmoid of kernels/prepare_gated_i8.loom:97-101 and
 * kernels/gemm_i8_swiglu_256.loom:649-652. The reference evaluates
 * `expf<afn>`, whose approximation belongs to its compiler; this build fixes its
 * own: Cody-Waite reduction x = n ln2 + r with a two-part ln2, then
 * 1 + r + r^2 q(r) with q a degree-4 Chebyshev-weighted least-squares fit of
 * (e^r - 1 - r)/r^2 on [-ln2/2, ln2/2], then 2^n applied as two exact power-of-two
 * factors. The device code evaluates the same function (its steps differ only in
 * ways that leave every result unchanged: one ldexp for 2^n, selected special
 * cases, and a corrected hardware reciprocal for 1/den); the GPU tests compare the
 * device sigmoid with this one bit for bit over the f32 range.
 */
float ora_expf(float x) {
    if (x != x) return x;
    if (x > 0x1.62e42ep+6f) return INFINITY; /* 88.72283 */
    if (x < -0x1.9fe368p+6f) return 0.0f;    /* -103.97208 */
    float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(n, -0x1.62e4p-1f, x);
    r = fmaf(n, -0x1.7f7d1cp-20f, r);
    float q = fmaf(0x1.6d4854p-10f, r, 0x1.121286p-7f);
    q = fmaf(q, r, 0x1.5554e6p-5f);
    q = fmaf(q, r, 0x1.5554d6p-3f);
    q = fmaf(q, r, 0.5f);
    float r2 = r * r;
    float p = 1.0f + fmaf(q, r2, r);
    int ni = (int)n;
    int n1 = ni / 2;
    int n2 = ni - n1;
    float s1 = float_of((uint32_t)(n1 + 127) << 23);
    float s2 = float_of((uint32_t)(n2 + 127) << 23);
    return (p * s1) * s2;
}

void ora_expf_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = ora_expf(x[i]);
}
/* sigmoid(g) = 1 / (1 + exp(-g)) with this file's exp and IEEE f32 division: the
 * function of kernels/prepare_gated_i8.loom:97-101 and kernels/gemm_i8_swiglu_256.loom:
 * 649-652 with expf<afn> replaced by ora_expf. Bit patterns of all 2^32 inputs from
 * `first` on are generated here (y[i] = sigmoid(bits first + i)), multithreaded. */
void ora_sigmoid_bits_n(uint32_t first, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t b = first + (uint32_t)i;
        float g;
        memcpy(&g, &b, 4);
        y[i] = 1.0f / (1.0f + ora_expf(0.0f - g));
    }
}

void ora_f16_from_f32_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = ora_f16_from_f32(x[i]);
}
void ora_bf16_from_f32_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = ora_bf16_from_f32(x[i]);
}

int ora_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static int pick_threads(int threads) {
    int t = threads > 0 ? threads : ora_max_threads();
    return t < 1 ? 1 : t;
}

/*
 * One radix-4 stage of the regular Hadamard H4 = [[1,1,1,-1],[1,1,-1,1],
 * [1,-1,1,1],[-1,1,1,1]] over quads (b, b+s, b+2s, b+3s) inside blocks of 4s,
 * in the reference's operation order (kernels/prepare_norm_i8.loom:190-205):
 *   s01 = e0+e1, s23 = e2+e3, d01 = e0-e1, d23 = e2-e3,
 *   o0 = s01+d23, o1 = s01-d23, o2 = d01+s23, o3 = s23-d01.
 * `f16_quarter` selects the plain prepare's stage rounding f16(0.25*o)
 * (kernels/prepare_plain_i8.loom:112-127,213-232).
 */
static void hadamard_stage(float *x, int64_t width, int64_t s, int f16_quarter) {
    for (int64_t block = 0; block < width; block += 4 * s) {
        for (int64_t col = 0; col < s; ++col) {
            float *p = x + block + col;
            float e0 = p[0], e1 = p[s], e2 = p[2 * s], e3 = p[3 * s];
            float s01 = e0 + e1, s23 = e2 + e3, d01 = e0 - e1, d23 = e2 - e3;
            float o0 = s01 + d23, o1 = s01 - d23, o2 = d01 + s23, o3 = s23 - d01;
            if (f16_quarter) {
                o0 = f16_round(o0 * 0.25f);
                o1 = f16_round(o1 * 0.25f);
                o2 = f16_round(o2 * 0.25f);
                o3 = f16_round(o3 * 0.25f);
            }
            p[0] = o0;
            p[s] = o1;
            p[2 * s] = o2;
            p[3 * s] = o3;
        }
    }
}

static void rotate(float *x, int64_t width, int f16_quarter) {
    hadamard_stage(x, width, 1, f16_quarter);
    hadamard_stage(x, width, 4, f16_quarter);
    hadamard_stage(x, width, 16, f16_quarter);
    hadamard_stage(x, width, 64, f16_quarter);
}

/*
 * Per-token symmetric quantisation, kernels/prepare_plain_i8.loom:283-346 and
 * kernels/prepare_norm_i8.loom:312-373: amax of |x|, row_max = amax * rs,
 * s = max(row_max, 1e-30)/127, inv = rs/s, q = clamp(rne(x*inv), +-127), where
 * rs = 16 for the plain prepare (its stages divided by 4 each) and 1/16 for the
 * f32 prepares (unscaled stages).
 */
static void quantise(const float *x, int64_t width, float rotation_scale, int8_t *q,
                     float *scale) {
    float amax = 0.0f;
    for (int64_t i = 0; i < width; ++i) amax = fmaxf(amax, fabsf(x[i]));
    float row_max = amax * rotation_scale;
    float safe = fmaxf(row_max, 1e-30f);
    float s = safe / 127.0f;
    float inv = rotation_scale / s;
    for (int64_t i = 0; i < width; ++i) {
        float v = rintf(x[i] * inv);
        v = fmaxf(v, -127.0f);
        v = fminf(v, 127.0f);
        q[i] = (int8_t)(int)v;
    }
    *scale = s;
}

/* kernels/prepare_plain_i8.loom:1-348 */
void ora_prepare_plain_i8(int64_t tokens, int64_t width, int64_t out_stride,
                          const uint16_t *h, int8_t *q, float *q_scale, int threads) {
    int nt = pick_threads(threads);
#pragma omp parallel num_threads(nt)
    {
    float *row = (float *)malloc((size_t)width * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t i = 0; i < width; ++i) row[i] = ora_f16_to_f32(h[t * width + i]);
        rotate(row, width, 1);
        quantise(row, width, 16.0f, q + t * out_stride, q_scale + t);
    }
    free(row);
    }
}

/*
 * The canonical sum of squares. The reference (kernels/prepare_norm_i8.loom:90-138)
 * runs 256 lanes; lane L keeps eight partial sums acc[e] over its chunks
 * c = L, L+256, ... (elements 8c+e), reduces them (`vector.reduce`), then each
 * 32-lane wave reduces its lanes (`subgroup.reduce`), and the eight wave sums are
 * combined as ((p0+p4)+(p2+p6))+((p1+p5)+(p3+p7)). The first two orders are the
 * reference compiler's; this build fixes them as: acc[e] accumulated in chunk
 * order, acc reduced left to right starting from 0, and the 32 lanes reduced by
 * an xor butterfly with strides 1, 2, 4, 8, 16 (lane l adds lane l^stride).
 */
float ora_norm_sum_squares(int64_t width, const uint16_t *h_row) {
    float lane_sum[256];
    int64_t chunks = width / 8;
    for (int lane = 0; lane < 256; ++lane) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t c = lane; c < chunks; c += 256) {
            for (int e = 0; e < 8; ++e) {
                float x = ora_bf16_to_f32(h_row[c * 8 + e]);
                float sq = x * x;
                acc[e] = acc[e] + sq;
            }
        }
        float s = 0.0f;
        for (int e = 0; e < 8; ++e) s = s + acc[e];
        lane_sum[lane] = s;
    }
    float p[8];
    for (int w = 0; w < 8; ++w) {
        float v[32];
        for (int l = 0; l < 32; ++l) v[l] = lane_sum[w * 32 + l];
        for (int stride = 1; stride < 32; stride *= 2) {
            float nv[32];
            for (int l = 0; l < 32; ++l) nv[l] = v[l] + v[l ^ stride];
            memcpy(v, nv, sizeof v);
        }
        p[w] = v[0];
    }
    float pair0 = p[0] + p[4], pair1 = p[1] + p[5], pair2 = p[2] + p[6], pair3 = p[3] + p[7];
    float even = pair0 + pair2, odd = pair1 + pair3;
    return even + odd;
}

/* kernels/prepare_norm_i8.loom:1-375 */
void ora_prepare_norm_i8(int64_t tokens, int64_t width, int64_t out_stride, float eps,
                         const uint16_t *h, const float *norm_scale, const float *mod_scale,
                         const float *mod_shift, int8_t *q, float *q_scale, int threads) {
    int nt = pick_threads(threads);
#pragma omp parallel num_threads(nt)
    {
    float *row = (float *)malloc((size_t)width * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        const uint16_t *hr = h + t * width;
        float total = ora_norm_sum_squares(width, hr);
        float mean = total / (float)width;
        float mean_eps = mean + eps;
        /* reference: rsqrtf (compiler-defined); canonical: correctly rounded 1/sqrt */
        float rms_inv = 1.0f / sqrtf(mean_eps);
        for (int64_t i = 0; i < width; ++i) { /* :145-170 */
            float x = ora_bf16_to_f32(hr[i]);
            float n = x * rms_inv;
            float ns1 = norm_scale[i] + 1.0f;
            float normed = bf_round(n * ns1);
            float ms1 = bf_round(mod_scale[i] + 1.0f);
            float scaled = bf_round(normed * ms1);
            row[i] = bf_round(scaled + mod_shift[i]);
        }
        rotate(row, width, 0);
        quantise(row, width, 0.0625f, q + t * out_stride, q_scale + t);
    }
    free(row);
    }
}

/* kernels/prepare_gated_i8.loom:1-313 (element formation :86-108) */
void ora_prepare_gated_i8(int64_t tokens, int64_t width, int64_t out_stride,
                          int64_t gate_stride, const uint16_t *attn, const uint16_t *gate,
                          int8_t *q, float *q_scale, int threads) {
    int nt = pick_threads(threads);
#pragma omp parallel num_threads(nt)
    {
    float *row = (float *)malloc((size_t)width * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        for (int64_t i = 0; i < width; ++i) {
            float a = bf_round(ora_f16_to_f32(attn[t * width + i]));
            float g = ora_f16_to_f32(gate[t * gate_stride + i]);
            float e = ora_expf(0.0f - g);
            float den = 1.0f + e;
            float sig = bf_round(1.0f / den);
            row[i] = bf_round(a * sig);
        }
        rotate(row, width, 0);
        quantise(row, width, 0.0625f, q + t * out_stride, q_scale + t);
    }
    free(row);
    }
}

/* tests/quantized.rs:203-211: the exact integer dot */
void ora_gemm_i32(int64_t m, int64_t n, int64_t k_size, int64_t k_stride, const int8_t *a,
                  const int8_t *w, int32_t *acc, int threads) {
    int nt = pick_threads(threads);
    const int64_t nb = 64;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) collapse(2)
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t c0 = 0; c0 < n; c0 += nb) {
            const int8_t *ar = a + r * k_stride;
            int64_t c1 = c0 + nb < n ? c0 + nb : n;
            for (int64_t c = c0; c < c1; ++c) {
                const int8_t *wr = w + c * k_stride;
                int32_t s = 0;
                for (int64_t k = 0; k < k_size; ++k) s += (int32_t)ar[k] * (int32_t)wr[k];
                acc[r * n + c] = s;
            }
        }
    }
}

/* kernels/gemm_i8_256.loom:606-626: f16(bf16((f32(acc) * ws[n]) * as[m])) */
static inline float plain_value(int32_t acc, float ws, float as) {
    float v = (float)acc * ws;
    return bf_round(v * as);
}

void ora_epilogue_plain(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                        const float *a_scale, uint16_t *c_f16) {
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c)
            c_f16[r * n + c] = ora_f16_from_f32(plain_value(acc[r * n + c], w_scale[c], a_scale[r]));
}

/* kernels/gemm_i8_resid_256.loom:615-635:
 * x = bf16(x + bf16(gate[n] * bf16((f32(acc) * ws[n]) * as[m]))) */
void ora_epilogue_resid(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                        const float *a_scale, const float *gate, uint16_t *x_bf16) {
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            float lin = plain_value(acc[r * n + c], w_scale[c], a_scale[r]);
            float gated = bf_round(lin * gate[c]);
            float prior = ora_bf16_to_f32(x_bf16[r * n + c]);
            x_bf16[r * n + c] = ora_bf16_from_f32(prior + gated);
        }
}

/* kernels/gemm_i8_swiglu_256.loom:618-660: gate/up columns interleaved in 16-column
 * groups; output o reads gate column (o/16)*32 + o%16 and up column +16. */
void ora_epilogue_swiglu(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                         const float *a_scale, uint16_t *c_f16) {
    int64_t half = n / 2;
    for (int64_t r = 0; r < m; ++r)
        for (int64_t o = 0; o < half; ++o) {
            int64_t gc = (o / 16) * 32 + o % 16, uc = gc + 16;
            float g = plain_value(acc[r * n + gc], w_scale[gc], a_scale[r]);
            float u = plain_value(acc[r * n + uc], w_scale[uc], a_scale[r]);
            float e = ora_expf(0.0f - g);
            float den = 1.0f + e;
            float sig = 1.0f / den;
            float silu = bf_round(g * sig);
            float prod = bf_round(silu * u);
            c_f16[r * half + o] = ora_f16_from_f32(prod);
        }
}

void ora_epilogue_bias(int64_t m, int64_t n, const int32_t *acc, const float *w_scale,
                       const float *a_scale, const uint16_t *bias_f16, uint16_t *c_f16) {
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            float v = ((float)acc[r * n + c] * w_scale[c]) * a_scale[r];
            float b = ora_f16_to_f32(bias_f16[c]);
            c_f16[r * n + c] = ora_f16_from_f32(bf_round(v + b));
        }
}

void ora_gemm_i8(int64_t m, int64_t n, int64_t k_size, int64_t k_stride, const int8_t *a,
                 const int8_t *w, const float *w_scale, const float *a_scale, uint16_t *c_f16,
                 int threads) {
    int nt = pick_threads(threads);
    const int64_t nb = 64;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) collapse(2)
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t c0 = 0; c0 < n; c0 += nb) {
            const int8_t *ar = a + r * k_stride;
            int64_t c1 = c0 + nb < n ? c0 + nb : n;
            for (int64_t c = c0; c < c1; ++c) {
                const int8_t *wr = w + c * k_stride;
                int32_t s = 0;
                for (int64_t k = 0; k < k_size; ++k) s += (int32_t)ar[k] * (int32_t)wr[k];
                c_f16[r * n + c] = ora_f16_from_f32(plain_value(s, w_scale[c], a_scale[r]));
            }
        }
    }
}

/* ---- The attention step ------------------------------------------------------ */

/* Sum of squares of one 128-channel head in this build's canonical order: sixteen
 * partials of eight channels, each ((x0^2+x1^2)+(x2^2+x3^2))+((x4^2+x5^2)+(x6^2+x7^2)),
 * combined by a butterfly over partial offsets 1, 2, 4, 8 (pairwise tree in index
 * order). The reference (kernels/rope_qknorm_f16.loom:109-113) reduces four channels per
 * lane and then across its wave in an order its compiler chooses. */
float ora_head_sum_squares(const uint16_t *h) {
    float part[16];
    for (int j = 0; j < 16; ++j) {
        float x[8];
        for (int e = 0; e < 8; ++e) x[e] = ora_f16_to_f32(h[8 * j + e]);
        part[j] = ((x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3])) +
                  ((x[4] * x[4] + x[5] * x[5]) + (x[6] * x[6] + x[7] * x[7]));
    }
    for (int d = 1; d < 16; d <<= 1)
        for (int j = 0; j < 16; j += 2 * d) part[j] = part[j] + part[j + d];
    return part[0];
}

/* kernels/rope_qknorm_f16.loom:73-154: x = bf16((h * r) * (1 + scale[c])) with
 * r = 1/sqrt(ss/128 + eps); pairs rotate as (x0 cos - x1 sin, x1 cos + x0 sin), rounded
 * to bf16 and stored as f16 (:128-146); v heads are copied (:90-94). */
void ora_rope_qknorm_f16(int64_t tokens, int64_t row_stride, int64_t q_heads, int64_t kv_heads,
                         int64_t k_offset, float eps, const uint16_t *qkv, const float *q_scale,
                         const float *k_scale, const float *cos_t, const float *sin_t,
                         uint16_t *q_out, uint16_t *k_out, uint16_t *v_out) {
    const int64_t heads = q_heads + 2 * kv_heads;
#pragma omp parallel for schedule(static)
    for (int64_t item = 0; item < tokens * heads; ++item) {
        const int64_t t = item / heads, head = item % heads;
        const uint16_t *row = qkv + t * row_stride;
        if (head >= q_heads + kv_heads) {
            const int64_t vh = head - q_heads - kv_heads;
            memcpy(v_out + (t * kv_heads + vh) * 128, row + k_offset + (kv_heads + vh) * 128, 256);
            continue;
        }
        const int is_q = head < q_heads;
        const int64_t kh = head - q_heads;
        const uint16_t *h = row + (is_q ? head * 128 : k_offset + kh * 128);
        const float *scale = is_q ? q_scale : k_scale;
        const float ss = ora_head_sum_squares(h);
        /* reference: rsqrtf (compiler-defined); canonical: correctly rounded 1/sqrt */
        const float rinv = 1.0f / sqrtf(ss * 0.0078125f + eps);
        float x[128];
        for (int c = 0; c < 128; ++c)
            x[c] = ora_bf16_to_f32(ora_bf16_from_f32((ora_f16_to_f32(h[c]) * rinv) * (scale[c] + 1.0f)));
        uint16_t *dst = is_q ? q_out + (t * q_heads + head) * 128 : k_out + (t * kv_heads + kh) * 128;
        const float *cs = cos_t + t * 128, *sn = sin_t + t * 128;
        for (int c = 0; c < 128; c += 2) {
            const float a = x[c] * cs[c] - x[c + 1] * sn[c];
            const float b = x[c + 1] * cs[c + 1] + x[c] * sn[c + 1];
            dst[c] = ora_f16_from_f32(ora_bf16_to_f32(ora_bf16_from_f32(a)));
            dst[c + 1] = ora_f16_from_f32(ora_bf16_to_f32(ora_bf16_from_f32(b)));
        }
    }
}

/* kernels/native/v_transpose.loom:48-88 */
void ora_v_transpose(int64_t rows, int64_t width, int64_t capacity, const uint16_t *x,
                     uint16_t *out) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < width; ++c) out[c * capacity + r] = x[r * width + c];
}

/* kernels/attention_gqa_lds_f16_wmma.loom:170-335: for each query row and head, scores
 * s_j = scale * (q . k_j) with f32 products of f16 values, keys j >= tokens excluded;
 * per key tile the running max m moves to max(m, tile max), the running sum and the
 * accumulators are scaled by exp(m_old - m_new), each weight w_j = exp(s_j - m_new) is
 * added to the sum in f32 and, rounded to f16, multiplies v_j into the accumulators;
 * out = f16(acc / sum) (:337-379). */
void ora_attention_f16(int64_t tokens, int64_t rows_out, int64_t capacity, int64_t q_stride,
                       int64_t kv_stride, int64_t out_stride, int64_t kv_heads, int64_t group,
                       float scale, int64_t key_tile, const uint16_t *q, const uint16_t *k,
                       const uint16_t *vt, uint16_t *out, int threads) {
    const int nt = threads > 0 ? threads : ora_max_threads();
    const int64_t heads = group * kv_heads;
    const int64_t rows = rows_out < tokens ? rows_out : tokens;
#pragma omp parallel num_threads(nt)
    {
        float *s = malloc(sizeof(float) * (size_t)key_tile);
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t t = 0; t < rows; ++t) {
                const int64_t kvh = h / group;
                float qv[128], acc[128];
                for (int c = 0; c < 128; ++c) {
                    qv[c] = ora_f16_to_f32(q[t * q_stride + h * 128 + c]);
                    acc[c] = 0.0f;
                }
                float m = -INFINITY, sum = 0.0f;
                for (int64_t j0 = 0; j0 < tokens; j0 += key_tile) {
                    const int64_t n = tokens - j0 < key_tile ? tokens - j0 : key_tile;
                    float tmax = -INFINITY;
                    for (int64_t j = 0; j < n; ++j) {
                        const uint16_t *kr = k + (j0 + j) * kv_stride + kvh * 128;
                        float dot = 0.0f;
                        for (int c = 0; c < 128; ++c) dot += qv[c] * ora_f16_to_f32(kr[c]);
                        s[j] = dot * scale;
                        if (s[j] > tmax) tmax = s[j];
                    }
                    const float m_new = m > tmax ? m : tmax;
                    const float alpha = expf(m - m_new);
                    sum *= alpha;
                    for (int c = 0; c < 128; ++c) acc[c] *= alpha;
                    for (int64_t j = 0; j < n; ++j) {
                        const float w = expf(s[j] - m_new);
                        sum += w;
                        const float w16 = ora_f16_to_f32(ora_f16_from_f32(w));
                        for (int c = 0; c < 128; ++c)
                            acc[c] += w16 * ora_f16_to_f32(vt[(kvh * 128 + c) * capacity + j0 + j]);
                    }
                    m = m_new;
                }
                for (int c = 0; c < 128; ++c)
                    out[t * out_stride + h * 128 + c] = ora_f16_from_f32(acc[c] / sum);
            }
        free(s);
    }
}
