/*
 * orc_core.c — CPU oracle: number formats, quantizers, dot products and the
 * encoder's operators.  TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * Every function restates one piece of ggml's CPU arithmetic as reached from
 * sam3.cpp's encoder graph.  ggml is absent from the reference mount
 * (.gitmodules:1-3, empty ggml/), so the ggml-internal steps are restated
 * from ggml's public MIT-licensed CPU sources ("[ext]" below) and pinned by
 * the checks named next to each function (tests/test_oracle_*.py):
 *
 *   fp16 conversion ........ exhaustive vs numpy float16 (RNE) — pinned
 *   q4_0/q4_1/q8_0 ref quant  closed-form reconstruction bounds + hand
 *                             fixtures in tests/golden — pinned
 *   q8_0/q8_1 SIMD quant .... tie fixtures (x·127/amax exactly k+0.5) fix the
 *                             RNE rounding; amax element maps to ±127 — pinned
 *   block dot products ...... int64 brute force of per-block sums and f64
 *                             dequantised dot — pinned
 *   mul_mat ................. f64 GEMM of dequantised operands — pinned
 *   layer norm / gelu_erf ... f64 numpy formulas — pinned
 *   rope .................... closed form sam3.cpp:3667-3706, axial cis KAT
 *                             tests/test_phase3.cpp:118-178 — pinned
 *   flash_attn_ext .......... f64 textbook softmax(QKᵀ·s)V, V=1 → O=1,
 *                             key-permutation invariance — pinned
 *
 * Build with -ffp-contract=off: every fused multiply-add below is written
 * out explicitly where ggml's SIMD code uses one.
 */
#include "orc.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#include <omp.h>

#define QK 32

/* ggml block structs (ggml-common.h [ext]); the file format stores exactly
 * these bytes (sam3.cpp:3131-3143, examples/quantize.cpp:244-262). */
typedef struct { uint16_t d; uint8_t qs[QK / 2]; } blk_q4_0;            /* 18 B */
typedef struct { uint16_t d; uint16_t m; uint8_t qs[QK / 2]; } blk_q4_1; /* 20 B */
typedef struct { uint16_t d; int8_t qs[QK]; } blk_q8_0;                  /* 34 B */
typedef struct { uint16_t d; uint16_t s; int8_t qs[QK]; } blk_q8_1;      /* 36 B */

_Static_assert(sizeof(blk_q4_0) == 18, "q4_0 size");
_Static_assert(sizeof(blk_q4_1) == 20, "q4_1 size");
_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 size");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1 size");

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32.  ggml on x86 with F16C uses _cvtss_sh(x, 0): IEEE binary16,
 * round to nearest even [ext].  Written out in integer arithmetic so the
 * oracle does not depend on the host having F16C. */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: binary16 subnormal or zero */
        float a;
        memcpy(&a, &ax, 4);
        /* a·2^24 is exact; nearbyintf rounds half to even in the default mode. */
        const uint32_t r = (uint32_t)nearbyintf(a * 16777216.0f);
        return (uint16_t)(sign | r);
    }
    const uint32_t mant = ax & 0x7fffffu;
    const uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t h = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h++;
    }
    return (uint16_t)(sign | h);
}

/* Software fp16 → fp32 (exact); the tests compare it with F16C and numpy. */
float orc_fp16_to_fp32_soft(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m · 2^-24, exact in fp32 */
            float v = (float)m * (1.0f / 16777216.0f);
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* fp16 → fp32 is exact, so the F16C instruction gives the same value as the
 * software conversion above; it is used in the dot-product hot loops. */
float orc_fp16_to_fp32(uint16_t h) { return _cvtsh_ss(h); }

void orc_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp32_to_fp16(x[i]);
}

void orc_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------------ */
int64_t orc_blck_size(int type) {
    switch (type) {
        case ORC_TYPE_Q4_0: case ORC_TYPE_Q4_1: case ORC_TYPE_Q8_0: case ORC_TYPE_Q8_1: return QK;
        default: return 1;
    }
}

size_t orc_type_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: return 4;
        case ORC_TYPE_F16: return 2;
        case ORC_TYPE_Q4_0: return sizeof(blk_q4_0);
        case ORC_TYPE_Q4_1: return sizeof(blk_q4_1);
        case ORC_TYPE_Q8_0: return sizeof(blk_q8_0);
        case ORC_TYPE_Q8_1: return sizeof(blk_q8_1);
        default: return 0;
    }
}

size_t orc_row_size(int type, int64_t ne0) {
    return orc_type_size(type) * (size_t)(ne0 / orc_blck_size(type));
}

/* ggml-cpu type traits [ext]: q4_0, q8_0 → q8_0; q4_1 → q8_1; f16 → f16; f32 → f32. */
int orc_vec_dot_type(int wtype) {
    switch (wtype) {
        case ORC_TYPE_Q4_0: return ORC_TYPE_Q8_0;
        case ORC_TYPE_Q8_0: return ORC_TYPE_Q8_0;
        case ORC_TYPE_Q4_1: return ORC_TYPE_Q8_1;
        case ORC_TYPE_F16:  return ORC_TYPE_F16;
        default:            return ORC_TYPE_F32;
    }
}

/* ------------------------------------------------------------------------ */
/* Weight quantizers: ggml_quantize_chunk → quantize_row_*_ref, no imatrix,
 * as called by examples/quantize.cpp:244-245 [ext]. */
void orc_quantize_row_q4_0_ref(const float *x, void *vy, int64_t k) {
    blk_q4_0 *y = (blk_q4_0 *)vy;
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK; j++) {
            const float v = x[i * QK + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK / 2; ++j) {
            const float x0 = x[i * QK + j] * id;
            const float x1 = x[i * QK + QK / 2 + j] * id;
            int8_t t0 = (int8_t)(x0 + 8.5f);
            int8_t t1 = (int8_t)(x1 + 8.5f);
            const uint8_t xi0 = (uint8_t)(t0 < 15 ? t0 : 15);
            const uint8_t xi1 = (uint8_t)(t1 < 15 ? t1 : 15);
            y[i].qs[j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

void orc_quantize_row_q4_1_ref(const float *x, void *vy, int64_t k) {
    blk_q4_1 *y = (blk_q4_1 *)vy;
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        float min = FLT_MAX, max = -FLT_MAX;
        for (int j = 0; j < QK; j++) {
            const float v = x[i * QK + j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / ((1 << 4) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        y[i].m = orc_fp32_to_fp16(min);
        for (int j = 0; j < QK / 2; ++j) {
            const float x0 = (x[i * QK + j] - min) * id;
            const float x1 = (x[i * QK + QK / 2 + j] - min) * id;
            int8_t t0 = (int8_t)(x0 + 0.5f);
            int8_t t1 = (int8_t)(x1 + 0.5f);
            const uint8_t xi0 = (uint8_t)(t0 < 15 ? t0 : 15);
            const uint8_t xi1 = (uint8_t)(t1 < 15 ? t1 : 15);
            y[i].qs[j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

void orc_quantize_row_q8_0_ref(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) {
            const float v = fabsf(x[i * QK + j]);
            amax = amax > v ? amax : v;
        }
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK; ++j) {
            y[i].qs[j] = (int8_t)roundf(x[i * QK + j] * id);
        }
    }
}

void orc_quantize_row_q8_1_ref(const float *x, void *vy, int64_t k) {
    blk_q8_1 *y = (blk_q8_1 *)vy;
    const int64_t nb = k / QK;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) {
            const float v = fabsf(x[i * QK + j]);
            amax = amax > v ? amax : v;
        }
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        int sum = 0;
        for (int j = 0; j < QK; ++j) {
            y[i].qs[j] = (int8_t)roundf(x[i * QK + j] * id);
            sum += y[i].qs[j];
        }
        y[i].s = orc_fp32_to_fp16((float)sum * d);
    }
}

/* Which of ggml's CPU builds the quantized products, the activation
 * quantizers and the f32 dots restate (orc_set_variant). */
static int g_variant = ORC_VARIANT_X86;
void orc_set_variant(int v) { g_variant = v; }
static inline int arm_variant(void) {
    return g_variant == ORC_VARIANT_ARM || g_variant == ORC_VARIANT_ARM_DOTPROD || g_variant == ORC_VARIANT_ARM_I8MM;
}

/* Activation quantizers: ggml-cpu x86 quantize_row_q8_0 / q8_1 (AVX2 path)
 * [ext]: maxScalar = max|x| over the block, d = maxScalar/127,
 * id = maxScalar != 0 ? 127/maxScalar : 0, q = round-half-even(x·id)
 * (_mm256_round_ps(.., _MM_ROUND_NEAREST)), q8_1 adds s = fp16(d·Σq).
 * The ARM NEON build (arch/arm/quants.c [ext]) takes id = d != 0 ? 1/d : 0
 * instead — the same reciprocal in another rounding, so x·id can land on
 * the other side of a .5 — and rounds with vcvtnq_s32_f32 (half to even). */
static void quant_block_simd(const float *x, int8_t *q, float *d_out, int *sum_out) {
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) {
        const float v = fabsf(x[j]);
        amax = amax > v ? amax : v;
    }
    const float d = amax / 127.f;
    const float id = arm_variant() ? (d != 0.0f ? 1.0f / d : 0.0f) : ((amax != 0.0f) ? 127.f / amax : 0.0f);
    int sum = 0;
    for (int j = 0; j < QK; j++) {
        const float v = x[j] * id;
        const int qi = (int)nearbyintf(v); /* default rounding mode: half to even */
        q[j] = (int8_t)qi;
        sum += qi;
    }
    *d_out = d;
    *sum_out = sum;
}

void orc_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    for (int64_t i = 0; i < k / QK; i++) {
        float d; int sum;
        quant_block_simd(x + i * QK, y[i].qs, &d, &sum);
        y[i].d = orc_fp32_to_fp16(d);
    }
}

void orc_quantize_row_q8_1(const float *x, void *vy, int64_t k) {
    blk_q8_1 *y = (blk_q8_1 *)vy;
    for (int64_t i = 0; i < k / QK; i++) {
        float d; int sum;
        quant_block_simd(x + i * QK, y[i].qs, &d, &sum);
        y[i].d = orc_fp32_to_fp16(d);
        y[i].s = orc_fp32_to_fp16(d * (float)sum);
    }
}

void orc_from_float(int type, const float *x, void *y, int64_t k) {
    switch (type) {
        case ORC_TYPE_Q8_0: orc_quantize_row_q8_0(x, y, k); break;
        case ORC_TYPE_Q8_1: orc_quantize_row_q8_1(x, y, k); break;
        case ORC_TYPE_F16:  orc_fp32_to_fp16_row(x, (uint16_t *)y, k); break;
        case ORC_TYPE_F32:  memcpy(y, x, (size_t)k * 4); break;
        default: break;
    }
}

/* dequantize_row_* (ggml to_float) [ext]. */
void orc_dequantize_row(int type, const void *vx, float *y, int64_t k) {
    const int64_t nb = k / QK;
    switch (type) {
        case ORC_TYPE_F32: memcpy(y, vx, (size_t)k * 4); break;
        case ORC_TYPE_F16: orc_fp16_to_fp32_row((const uint16_t *)vx, y, k); break;
        case ORC_TYPE_Q4_0: {
            const blk_q4_0 *x = (const blk_q4_0 *)vx;
            for (int64_t i = 0; i < nb; i++) {
                const float d = orc_fp16_to_fp32(x[i].d);
                for (int j = 0; j < QK / 2; ++j) {
                    y[i * QK + j] = (float)((x[i].qs[j] & 0x0F) - 8) * d;
                    y[i * QK + j + QK / 2] = (float)((x[i].qs[j] >> 4) - 8) * d;
                }
            }
        } break;
        case ORC_TYPE_Q4_1: {
            const blk_q4_1 *x = (const blk_q4_1 *)vx;
            for (int64_t i = 0; i < nb; i++) {
                const float d = orc_fp16_to_fp32(x[i].d);
                const float m = orc_fp16_to_fp32(x[i].m);
                for (int j = 0; j < QK / 2; ++j) {
                    y[i * QK + j] = (float)(x[i].qs[j] & 0x0F) * d + m;
                    y[i * QK + j + QK / 2] = (float)(x[i].qs[j] >> 4) * d + m;
                }
            }
        } break;
        case ORC_TYPE_Q8_0: {
            const blk_q8_0 *x = (const blk_q8_0 *)vx;
            for (int64_t i = 0; i < nb; i++) {
                const float d = orc_fp16_to_fp32(x[i].d);
                for (int j = 0; j < QK; ++j) y[i * QK + j] = (float)x[i].qs[j] * d;
            }
        } break;
        case ORC_TYPE_Q8_1: {
            const blk_q8_1 *x = (const blk_q8_1 *)vx;
            for (int64_t i = 0; i < nb; i++) {
                const float d = orc_fp16_to_fp32(x[i].d);
                for (int j = 0; j < QK; ++j) y[i * QK + j] = (float)x[i].qs[j] * d;
            }
        } break;
        default: break;
    }
}

/* ------------------------------------------------------------------------ */
/* Dot products.  The AVX2 kernels of ggml-cpu (arch/x86/quants.c,
 * vec.cpp) [ext] accumulate one __m256 of eight fp32 lanes: for each block,
 * lane i receives d_w·d_x times the int32 sum of elements 4i..4i+3, through
 * an FMA; the eight lanes are reduced by hsum_float_8 at the end.  The code
 * below follows that order with the same intrinsics. */
static inline float hsum_float_8(const __m256 x) {
    __m128 res = _mm256_extractf128_ps(x, 1);
    res = _mm_add_ps(res, _mm256_castps256_ps128(x));
    res = _mm_add_ps(res, _mm_movehl_ps(res, res));
    res = _mm_add_ss(res, _mm_movehdup_ps(res));
    return _mm_cvtss_f32(res);
}

static inline __m256i bytes_from_nibbles_32(const uint8_t *rsi) {
    const __m128i tmp = _mm_loadu_si128((const __m128i *)rsi);
    const __m256i bytes = _mm256_insertf128_si256(_mm256_castsi128_si256(tmp), _mm_srli_epi16(tmp, 4), 1);
    const __m256i lowMask = _mm256_set1_epi8(0xF);
    return _mm256_and_si256(lowMask, bytes);
}

/* Σ of products of four consecutive signed bytes per int32 lane, as float. */
static inline __m256 mul_sum_i8_pairs_float(const __m256i x, const __m256i y) {
    const __m256i ax = _mm256_sign_epi8(x, x);
    const __m256i sy = _mm256_sign_epi8(y, x);
    const __m256i dot = _mm256_maddubs_epi16(ax, sy);
    const __m256i summed = _mm256_madd_epi16(_mm256_set1_epi16(1), dot);
    return _mm256_cvtepi32_ps(summed);
}

/* Same with x unsigned (q4_1 nibbles). */
static inline __m256 mul_sum_us8_pairs_float(const __m256i ax, const __m256i sy) {
    const __m256i dot = _mm256_maddubs_epi16(ax, sy);
    const __m256i summed = _mm256_madd_epi16(_mm256_set1_epi16(1), dot);
    return _mm256_cvtepi32_ps(summed);
}

static float vec_dot_q4_0_q8_0(int64_t n, const blk_q4_0 *x, const blk_q8_0 *y) {
    const int64_t nb = n / QK;
    __m256 acc = _mm256_setzero_ps();
    for (int64_t ib = 0; ib < nb; ++ib) {
        const __m256 d = _mm256_set1_ps(orc_fp16_to_fp32(x[ib].d) * orc_fp16_to_fp32(y[ib].d));
        __m256i qx = bytes_from_nibbles_32(x[ib].qs);
        qx = _mm256_sub_epi8(qx, _mm256_set1_epi8(8));
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256 q = mul_sum_i8_pairs_float(qx, qy);
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum_float_8(acc);
}

static float vec_dot_q8_0_q8_0(int64_t n, const blk_q8_0 *x, const blk_q8_0 *y) {
    const int64_t nb = n / QK;
    __m256 acc = _mm256_setzero_ps();
    for (int64_t ib = 0; ib < nb; ++ib) {
        const __m256 d = _mm256_set1_ps(orc_fp16_to_fp32(x[ib].d) * orc_fp16_to_fp32(y[ib].d));
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256 q = mul_sum_i8_pairs_float(qx, qy);
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum_float_8(acc);
}

static float vec_dot_q4_1_q8_1(int64_t n, const blk_q4_1 *x, const blk_q8_1 *y) {
    const int64_t nb = n / QK;
    __m256 acc = _mm256_setzero_ps();
    float summs = 0;
    for (int64_t ib = 0; ib < nb; ++ib) {
        const float d0 = orc_fp16_to_fp32(x[ib].d);
        const float d1 = orc_fp16_to_fp32(y[ib].d);
        summs = fmaf(orc_fp16_to_fp32(x[ib].m), orc_fp16_to_fp32(y[ib].s), summs);
        const __m256 d0d1 = _mm256_mul_ps(_mm256_set1_ps(d0), _mm256_set1_ps(d1));
        const __m256i qx = bytes_from_nibbles_32(x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256 xy = mul_sum_us8_pairs_float(qx, qy);
        acc = _mm256_fmadd_ps(d0d1, xy, acc);
    }
    return hsum_float_8(acc) + summs;
}

/* ggml_vec_dot_f16 / ggml_vec_dot_f32 with F16C+FMA [ext]: four __m256
 * accumulators over steps of 32 elements, FMA per step, GGML_F32x8_REDUCE,
 * then a scalar tail accumulated in double. */
static float reduce4(__m256 s[4]) {
    s[0] = _mm256_add_ps(s[0], s[2]);
    s[1] = _mm256_add_ps(s[1], s[3]);
    s[0] = _mm256_add_ps(s[0], s[1]);
    const __m128 t0 = _mm_add_ps(_mm256_castps256_ps128(s[0]), _mm256_extractf128_ps(s[0], 1));
    const __m128 t1 = _mm_hadd_ps(t0, t0);
    return _mm_cvtss_f32(_mm_hadd_ps(t1, t1));
}

static float vec_dot_f16(int64_t n, const uint16_t *x, const uint16_t *y) {
    const int64_t np = n & ~(int64_t)31;
    __m256 s[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (int64_t i = 0; i < np; i += 32) {
        for (int j = 0; j < 4; j++) {
            const __m256 ax = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x + i + j * 8)));
            const __m256 ay = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i + j * 8)));
            s[j] = _mm256_fmadd_ps(ax, ay, s[j]);
        }
    }
    double sumf = reduce4(s);
    for (int64_t i = np; i < n; ++i) {
        sumf += (double)(orc_fp16_to_fp32(x[i]) * orc_fp16_to_fp32(y[i]));
    }
    return (float)sumf;
}

static float vec_dot_f32(int64_t n, const float *x, const float *y) {
    const int64_t np = n & ~(int64_t)31;
    __m256 s[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (int64_t i = 0; i < np; i += 32) {
        for (int j = 0; j < 4; j++) {
            const __m256 ax = _mm256_loadu_ps(x + i + j * 8);
            const __m256 ay = _mm256_loadu_ps(y + i + j * 8);
            s[j] = _mm256_fmadd_ps(ax, ay, s[j]);
        }
    }
    double sumf = reduce4(s);
    for (int64_t i = np; i < n; ++i) {
        sumf += (double)(x[i] * y[i]);
    }
    return (float)sumf;
}

/* ggml's generic (non-SIMD) vec_dot paths [ext]: the same block math with a
 * different fp32 evaluation order — per block sumi·d_x·d_w (left to right)
 * added to a scalar float sum; F16/F32 accumulate each product in double.
 * Used only to measure how much ggml's own results move with the order. */
static float vec_dot_generic(int wtype, int64_t n, const void *w, const void *x) {
    const int64_t nb = n / QK;
    float sumf = 0.0f;
    if (wtype == ORC_TYPE_Q4_0 || wtype == ORC_TYPE_Q8_0) {
        int32_t s[4096];
        orc_block_isums(wtype, n, w, x, s);
        for (int64_t b = 0; b < nb; b++) {
            const float dw = orc_fp16_to_fp32(wtype == ORC_TYPE_Q4_0 ? ((const blk_q4_0 *)w)[b].d : ((const blk_q8_0 *)w)[b].d);
            const float dx = orc_fp16_to_fp32(((const blk_q8_0 *)x)[b].d);
            const float t = ((float)s[b] * dw) * dx;
            sumf = sumf + t;
        }
        return sumf;
    }
    if (wtype == ORC_TYPE_Q4_1) {
        int32_t s[4096];
        orc_block_isums(wtype, n, w, x, s);
        for (int64_t b = 0; b < nb; b++) {
            const blk_q4_1 *wb = (const blk_q4_1 *)w + b;
            const blk_q8_1 *xb = (const blk_q8_1 *)x + b;
            const float t0 = (orc_fp16_to_fp32(wb->d) * orc_fp16_to_fp32(xb->d)) * (float)s[b];
            const float t1 = orc_fp16_to_fp32(wb->m) * orc_fp16_to_fp32(xb->s);
            sumf = sumf + (t0 + t1);
        }
        return sumf;
    }
    double acc = 0.0;
    if (wtype == ORC_TYPE_F16) {
        for (int64_t i = 0; i < n; i++)
            acc += (double)(orc_fp16_to_fp32(((const uint16_t *)w)[i]) * orc_fp16_to_fp32(((const uint16_t *)x)[i]));
    } else {
        for (int64_t i = 0; i < n; i++) acc += (double)(((const float *)w)[i] * ((const float *)x)[i]);
    }
    return (float)acc;
}

/* ---- ARM NEON builds [ext] ------------------------------------------------
 * The reference's published CPU timings come from an Apple M4 Pro
 * (README.md:50-69), whose native build has the dotprod and i8mm
 * extensions.  There ggml_mul_mat reaches three block-dot orders:
 *
 *  - llamafile's tinyBLAS_Q0_ARM (sgemm.cpp), tried first for Q4_0 / Q8_0
 *    weights once src1 is in Q8_0: per output one float32x4 accumulator;
 *    per block, lane i gets fma(Σ_{j∈{4i..4i+3} ∪ {16+4i..16+4i+3}} w_j·x_j,
 *    d_w·d_x) (two vdotq_s32 over the block's low and high 16 bytes); the
 *    four lanes are summed pairwise at the end (vaddvq_f32).
 *  - ggml_vec_dot_*_q8_* with nrc = 2 (vmmlaq_s32, i8mm), used for Q4_1 and
 *    whenever the product has even row counts: per output one fp32 chain
 *    acc = fma(S_b, d_w·d_x, acc) over the exact block sums S_b; Q4_1 adds its
 *    Σ m_w·s_x in a second chain and the two are added at the end.
 *  - ggml_vec_dot_*_q8_* with nrc = 1 (dotprod only, e.g. without i8mm):
 *    the tinyBLAS lanes, but blocks alternate between two float32x4
 *    accumulators, vaddvq(sumv0) + vaddvq(sumv1) at the end; an odd last
 *    block is added as ((S_b·d_w)·d_x) fused into the sum; Q4_1 keeps
 *    Σ (m_w·s_x + m_w'·s_x') per block pair in one float added last.
 * vmlaq_n_f32 / vmlaq_f32 compile to fused multiply-adds under clang's and
 * gcc's default contraction, which is what is restated.  ORC_VARIANT_ARM is
 * the M4 Pro's mixture: tinyBLAS for Q4_0 / Q8_0, nrc = 2 for Q4_1.
 * The f32 dot (attention scores with F32 K, F32 convolutions) is
 * ggml_vec_dot_f32 on NEON: four float32x4 accumulators over steps of 16,
 * reduced (0+2, 1+3), then (0+1), then vaddvq_f32. */

/* Exact int32 partial sums of one block: lane i = Σ_{j=4i}^{4i+3} w_j·x_j. */
static inline __m256i block_p8(int wtype, const void *wb, const void *xb) {
    if (wtype == ORC_TYPE_Q4_1) {
        const __m256i qw = bytes_from_nibbles_32(((const blk_q4_1 *)wb)->qs);
        const __m256i qx = _mm256_loadu_si256((const __m256i *)((const blk_q8_1 *)xb)->qs);
        return _mm256_madd_epi16(_mm256_set1_epi16(1), _mm256_maddubs_epi16(qw, qx));
    }
    __m256i qw;
    if (wtype == ORC_TYPE_Q4_0) qw = _mm256_sub_epi8(bytes_from_nibbles_32(((const blk_q4_0 *)wb)->qs), _mm256_set1_epi8(8));
    else qw = _mm256_loadu_si256((const __m256i *)((const blk_q8_0 *)wb)->qs);
    const __m256i qx = _mm256_loadu_si256((const __m256i *)((const blk_q8_0 *)xb)->qs);
    const __m256i dot = _mm256_maddubs_epi16(_mm256_sign_epi8(qw, qw), _mm256_sign_epi8(qx, qw));
    return _mm256_madd_epi16(_mm256_set1_epi16(1), dot);
}

static inline float vaddv4(const float a[4]) { return (a[0] + a[1]) + (a[2] + a[3]); }

/* One (weight row, activation row) product in the ARM orders. */
static float vec_dot_arm(int variant, int wtype, int64_t n, const char *w, const char *x) {
    const int64_t nb = n / QK;
    const size_t wbs = wtype == ORC_TYPE_Q4_0 ? sizeof(blk_q4_0) : wtype == ORC_TYPE_Q4_1 ? sizeof(blk_q4_1) : sizeof(blk_q8_0);
    const size_t xbs = wtype == ORC_TYPE_Q4_1 ? sizeof(blk_q8_1) : sizeof(blk_q8_0);
    const int q41 = wtype == ORC_TYPE_Q4_1;
    if (variant == ORC_VARIANT_ARM) variant = q41 ? ORC_VARIANT_ARM_I8MM : -1; /* -1: tinyBLAS */
    float acc = 0.0f, summs = 0.0f;
    float v[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    int64_t b = 0;
    const int64_t npair = variant == ORC_VARIANT_ARM_DOTPROD ? nb & ~(int64_t)1 : nb;
    for (; b < npair; b++) {
        const char *wb = w + b * wbs, *xb = x + b * xbs;
        const uint16_t wd = *(const uint16_t *)wb, xd = *(const uint16_t *)xb;
        const float d = orc_fp16_to_fp32(wd) * orc_fp16_to_fp32(xd);
        int32_t p[8];
        _mm256_storeu_si256((__m256i *)p, block_p8(wtype, wb, xb));
        if (variant == ORC_VARIANT_ARM_I8MM) {
            const int32_t S = p[0] + p[1] + p[2] + p[3] + p[4] + p[5] + p[6] + p[7];
            acc = fmaf((float)S, d, acc);
            if (q41) summs = summs + orc_fp16_to_fp32(((const blk_q4_1 *)wb)->m) * orc_fp16_to_fp32(((const blk_q8_1 *)xb)->s);
        } else {
            float *a = v[variant == ORC_VARIANT_ARM_DOTPROD ? (b & 1) : 0];
            for (int i = 0; i < 4; i++) a[i] = fmaf((float)(p[i] + p[i + 4]), d, a[i]);
            if (q41 && (b & 1)) {
                const blk_q4_1 *w0 = (const blk_q4_1 *)(wb - wbs), *w1 = (const blk_q4_1 *)wb;
                const blk_q8_1 *x0 = (const blk_q8_1 *)(xb - xbs), *x1 = (const blk_q8_1 *)xb;
                const float t = orc_fp16_to_fp32(w0->m) * orc_fp16_to_fp32(x0->s) +
                                orc_fp16_to_fp32(w1->m) * orc_fp16_to_fp32(x1->s);
                summs = summs + t;
            }
        }
    }
    float sumf;
    if (variant == ORC_VARIANT_ARM_I8MM) return q41 ? acc + summs : acc;
    if (variant == ORC_VARIANT_ARM_DOTPROD) {
        sumf = vaddv4(v[0]) + vaddv4(v[1]);
        if (q41) sumf = sumf + summs;
        for (; b < nb; b++) { /* odd last block: the scalar tail */
            const char *wb = w + b * wbs, *xb = x + b * xbs;
            int32_t S = 0;
            orc_block_isums(wtype, QK, wb, xb, &S);
            const float dw = orc_fp16_to_fp32(*(const uint16_t *)wb), dx = orc_fp16_to_fp32(*(const uint16_t *)xb);
            if (q41) {
                const float t = fmaf(dw * dx, (float)S, orc_fp16_to_fp32(((const blk_q4_1 *)wb)->m) *
                                                           orc_fp16_to_fp32(((const blk_q8_1 *)xb)->s));
                sumf = sumf + t;
            } else {
                sumf = fmaf((float)S * dw, dx, sumf);
            }
        }
        return sumf;
    }
    return vaddv4(v[0]); /* tinyBLAS_Q0_ARM: hsum of the one accumulator */
}

/* ggml_vec_dot_f32 on NEON (GGML_F32_STEP 16, four float32x4 accumulators). */
static float vec_dot_f32_neon(int64_t n, const float *x, const float *y) {
    const int64_t np = n & ~(int64_t)15;
    float s[4][4] = {{0}};
    for (int64_t i = 0; i < np; i += 16)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 4; l++) s[j][l] = fmaf(x[i + 4 * j + l], y[i + 4 * j + l], s[j][l]);
    for (int l = 0; l < 4; l++) {
        s[0][l] = s[0][l] + s[2][l];
        s[1][l] = s[1][l] + s[3][l];
    }
    for (int l = 0; l < 4; l++) s[0][l] = s[0][l] + s[1][l];
    float sumf = vaddv4(s[0]);
    for (int64_t i = np; i < n; ++i) sumf = fmaf(x[i], y[i], sumf);
    return sumf;
}

float orc_vec_dot(int wtype, int64_t n, const void *w, const void *x) {
    if (g_variant == ORC_VARIANT_GENERIC && n / QK <= 4096) return vec_dot_generic(wtype, n, w, x);
    if (arm_variant()) {
        if (wtype == ORC_TYPE_Q4_0 || wtype == ORC_TYPE_Q8_0 || wtype == ORC_TYPE_Q4_1)
            return vec_dot_arm(g_variant, wtype, n, (const char *)w, (const char *)x);
        if (wtype == ORC_TYPE_F32) return vec_dot_f32_neon(n, (const float *)w, (const float *)x);
    }
    switch (wtype) {
        case ORC_TYPE_Q4_0: return vec_dot_q4_0_q8_0(n, (const blk_q4_0 *)w, (const blk_q8_0 *)x);
        case ORC_TYPE_Q8_0: return vec_dot_q8_0_q8_0(n, (const blk_q8_0 *)w, (const blk_q8_0 *)x);
        case ORC_TYPE_Q4_1: return vec_dot_q4_1_q8_1(n, (const blk_q4_1 *)w, (const blk_q8_1 *)x);
        case ORC_TYPE_F16:  return vec_dot_f16(n, (const uint16_t *)w, (const uint16_t *)x);
        case ORC_TYPE_F32:  return vec_dot_f32(n, (const float *)w, (const float *)x);
        default: return NAN;
    }
}

/* Per-block integer sums, written with plain scalar loops (a second, independent
 * derivation of the block contents used by the exactness tests). */
void orc_block_isums(int wtype, int64_t n, const void *w, const void *x, int32_t *out) {
    const int64_t nb = n / QK;
    for (int64_t b = 0; b < nb; b++) {
        int32_t s = 0;
        if (wtype == ORC_TYPE_Q4_0) {
            const blk_q4_0 *wb = (const blk_q4_0 *)w + b;
            const blk_q8_0 *xb = (const blk_q8_0 *)x + b;
            for (int j = 0; j < QK / 2; j++) {
                s += ((wb->qs[j] & 15) - 8) * xb->qs[j];
                s += ((wb->qs[j] >> 4) - 8) * xb->qs[j + QK / 2];
            }
        } else if (wtype == ORC_TYPE_Q4_1) {
            const blk_q4_1 *wb = (const blk_q4_1 *)w + b;
            const blk_q8_1 *xb = (const blk_q8_1 *)x + b;
            for (int j = 0; j < QK / 2; j++) {
                s += (wb->qs[j] & 15) * xb->qs[j];
                s += (wb->qs[j] >> 4) * xb->qs[j + QK / 2];
            }
        } else if (wtype == ORC_TYPE_Q8_0) {
            const blk_q8_0 *wb = (const blk_q8_0 *)w + b;
            const blk_q8_0 *xb = (const blk_q8_0 *)x + b;
            for (int j = 0; j < QK; j++) s += wb->qs[j] * xb->qs[j];
        }
        out[b] = s;
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_mul_mat on the CPU backend [ext]: src1 (f32) is converted row by row
 * to the vec_dot type of src0, then each output element is one vec_dot of a
 * src0 row with a converted src1 row.  Called from the ViT block at
 * sam3.cpp:3738, 3779, 3792, 3795. */
/* 4×4 block of q4_0/q8_0/q4_1 dot products evaluated together: every one of
 * the 16 dots keeps exactly the per-dot order of the vec_dot kernels above
 * (one 8-lane accumulator, one FMA per block, hsum at the end), so results
 * are bit-identical to 16 separate vec_dot calls; loading each block once
 * for 4 dots only saves time. */
static void dot4x4_q(int wtype, int64_t K, const char *W, size_t wrs, const char *X, size_t xrs, float *Y,
                     int64_t ldy) {
    const int64_t nb = K / QK;
    __m256 acc[4][4];
    float summs[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) { acc[i][j] = _mm256_setzero_ps(); summs[i][j] = 0.0f; }
    for (int64_t b = 0; b < nb; b++) {
        __m256i qw[4], qx[4];
        float dw[4], dx[4], mw[4] = {0, 0, 0, 0}, sx[4] = {0, 0, 0, 0};
        for (int j = 0; j < 4; j++) {
            const char *wr = W + (size_t)j * wrs;
            if (wtype == ORC_TYPE_Q4_0) {
                const blk_q4_0 *wb = (const blk_q4_0 *)wr + b;
                dw[j] = orc_fp16_to_fp32(wb->d);
                qw[j] = _mm256_sub_epi8(bytes_from_nibbles_32(wb->qs), _mm256_set1_epi8(8));
            } else if (wtype == ORC_TYPE_Q4_1) {
                const blk_q4_1 *wb = (const blk_q4_1 *)wr + b;
                dw[j] = orc_fp16_to_fp32(wb->d);
                mw[j] = orc_fp16_to_fp32(wb->m);
                qw[j] = bytes_from_nibbles_32(wb->qs);
            } else {
                const blk_q8_0 *wb = (const blk_q8_0 *)wr + b;
                dw[j] = orc_fp16_to_fp32(wb->d);
                qw[j] = _mm256_loadu_si256((const __m256i *)wb->qs);
            }
        }
        for (int i = 0; i < 4; i++) {
            const char *xr = X + (size_t)i * xrs;
            if (wtype == ORC_TYPE_Q4_1) {
                const blk_q8_1 *xb = (const blk_q8_1 *)xr + b;
                dx[i] = orc_fp16_to_fp32(xb->d);
                sx[i] = orc_fp16_to_fp32(xb->s);
                qx[i] = _mm256_loadu_si256((const __m256i *)xb->qs);
            } else {
                const blk_q8_0 *xb = (const blk_q8_0 *)xr + b;
                dx[i] = orc_fp16_to_fp32(xb->d);
                qx[i] = _mm256_loadu_si256((const __m256i *)xb->qs);
            }
        }
        for (int i = 0; i < 4; i++)
            for (int j = 0; j < 4; j++) {
                if (wtype == ORC_TYPE_Q4_1) {
                    summs[i][j] = fmaf(mw[j], sx[i], summs[i][j]);
                    const __m256 d = _mm256_mul_ps(_mm256_set1_ps(dw[j]), _mm256_set1_ps(dx[i]));
                    acc[i][j] = _mm256_fmadd_ps(d, mul_sum_us8_pairs_float(qw[j], qx[i]), acc[i][j]);
                } else {
                    const __m256 d = _mm256_set1_ps(dw[j] * dx[i]);
                    acc[i][j] = _mm256_fmadd_ps(d, mul_sum_i8_pairs_float(qw[j], qx[i]), acc[i][j]);
                }
            }
    }
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            Y[i * ldy + j] = wtype == ORC_TYPE_Q4_1 ? hsum_float_8(acc[i][j]) + summs[i][j] : hsum_float_8(acc[i][j]);
}

void orc_mul_mat_preq(int wtype, const void *W, int64_t N, int64_t K,
                      const void *Xq, int64_t M, float *Y, int nthreads) {
    const int vdt = orc_vec_dot_type(wtype);
    const size_t wrs = orc_row_size(wtype, K);
    const size_t xrs = orc_row_size(vdt, K);
    const int64_t TM = 32, TN = 32;
    const int64_t tiles_m = (M + TM - 1) / TM, tiles_n = (N + TN - 1) / TN;
    const int blocked = g_variant == ORC_VARIANT_X86 &&
                        (wtype == ORC_TYPE_Q4_0 || wtype == ORC_TYPE_Q8_0 || wtype == ORC_TYPE_Q4_1);
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int64_t t = 0; t < tiles_m * tiles_n; t++) {
        const int64_t m0 = (t / tiles_n) * TM, n0 = (t % tiles_n) * TN;
        const int64_t m1 = m0 + TM < M ? m0 + TM : M;
        const int64_t n1 = n0 + TN < N ? n0 + TN : N;
        int64_t m = m0;
        if (blocked) {
            for (; m + 4 <= m1; m += 4) {
                int64_t n = n0;
                for (; n + 4 <= n1; n += 4) {
                    dot4x4_q(wtype, K, (const char *)W + (size_t)n * wrs, wrs, (const char *)Xq + (size_t)m * xrs,
                             xrs, Y + m * N + n, N);
                }
                for (int64_t mm = m; mm < m + 4; mm++)
                    for (int64_t nn = n; nn < n1; nn++)
                        Y[mm * N + nn] = orc_vec_dot(wtype, K, (const char *)W + (size_t)nn * wrs,
                                                     (const char *)Xq + (size_t)mm * xrs);
            }
        }
        for (; m < m1; m++) {
            const char *xr = (const char *)Xq + (size_t)m * xrs;
            for (int64_t n = n0; n < n1; n++) {
                Y[m * N + n] = orc_vec_dot(wtype, K, (const char *)W + (size_t)n * wrs, xr);
            }
        }
    }
}

void orc_mul_mat(int wtype, const void *W, int64_t N, int64_t K,
                 const float *X, int64_t M, float *Y, int nthreads) {
    const int vdt = orc_vec_dot_type(wtype);
    const size_t xrs = orc_row_size(vdt, K);
    char *Xq = (char *)malloc(xrs * (size_t)M);
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t m = 0; m < M; m++) {
        orc_from_float(vdt, X + m * K, Xq + (size_t)m * xrs, K);
    }
    orc_mul_mat_preq(wtype, W, N, K, Xq, M, Y, nthreads);
    free(Xq);
}

/* ------------------------------------------------------------------------ */
/* sam3_layer_norm (sam3.cpp:1037-1047) = ggml_norm(x, eps), ggml_mul_inplace(w),
 * ggml_add_inplace(b).  ggml_norm_f32 [ext]: mean accumulated in double and
 * rounded to float; centred values stored as float; variance accumulated in
 * double from the float squares; scale = 1/sqrtf(var + eps) in float. */
void orc_layer_norm(const float *x, float *y, int64_t rows, int64_t n, float eps,
                    const float *w, const float *b, int nthreads) {
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * n;
        float *yr = y + r * n;
        double sum = 0.0;
        for (int64_t i = 0; i < n; i++) sum += (double)xr[i];
        const float mean = (float)(sum / (double)n);
        double sum2 = 0.0;
        for (int64_t i = 0; i < n; i++) {
            const float v = xr[i] - mean;
            yr[i] = v;
            sum2 += (double)(v * v);
        }
        const float variance = (float)(sum2 / (double)n);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < n; i++) yr[i] *= scale;
        if (w) for (int64_t i = 0; i < n; i++) yr[i] = yr[i] * w[i];
        if (b) for (int64_t i = 0; i < n; i++) yr[i] = yr[i] + b[i];
    }
}

/* ggml_gelu_erf on f32 (ggml_vec_gelu_erf_f32) [ext]; used at sam3.cpp:3794. */
void orc_gelu_erf(float *x, int64_t n) {
    const float SQRT_2_INV = 0.70710678118654752440084436210484f;
    for (int64_t i = 0; i < n; i++) {
        const float xi = x[i];
        x[i] = 0.5f * xi * (1.0f + erff(xi * SQRT_2_INV));
    }
}

/* sam3_apply_rope (sam3.cpp:3667-3706): pairs (x[2i], x[2i+1]) rotated by
 * (cos, sin) = freqs[n][i]; each product and the sub/add are separate ggml
 * ops (ggml_mul, ggml_sub, ggml_add), so every step rounds on its own. */
void orc_rope(float *x, int64_t HD, int64_t N, int64_t nh, const float *freqs) {
    const int64_t half = HD / 2;
    for (int64_t h = 0; h < nh; h++) {
        for (int64_t n = 0; n < N; n++) {
            float *r = x + (h * N + n) * HD;
            const float *f = freqs + n * half * 2;
            for (int64_t i = 0; i < half; i++) {
                const float re = r[2 * i], im = r[2 * i + 1];
                const float c = f[2 * i], s = f[2 * i + 1];
                const float a = re * c, bb = im * s, cc = re * s, dd = im * c;
                r[2 * i] = a - bb;
                r[2 * i + 1] = cc + dd;
            }
        }
    }
}

/* ggml_flash_attn_ext CPU kernel (ggml_compute_forward_flash_attn_ext_f16,
 * one query row at a time) with F32 K/V, no mask [ext]; called at
 * sam3.cpp:3774 with scale = 1/sqrt(HD).  Per key: s = dot(q, k)·scale; if
 * s > M: M = s, ms = expf(Mold - M), VKQ *= ms, vs = 1; else vs = expf(s - M);
 * VKQ += v·vs (FMA); S = S·ms + vs.  Finally O = VKQ·(1/S). */
static void vec_mad_f32(int64_t n, float *y, const float *x, float v) {
    const int64_t np = n & ~(int64_t)31;
    const __m256 vx = _mm256_set1_ps(v);
    for (int64_t i = 0; i < np; i += 8) {
        _mm256_storeu_ps(y + i, _mm256_fmadd_ps(_mm256_loadu_ps(x + i), vx, _mm256_loadu_ps(y + i)));
    }
    for (int64_t i = np; i < n; i++) y[i] = fmaf(x[i], v, y[i]);
}

static void vec_scale_f32(int64_t n, float *y, float v) {
    for (int64_t i = 0; i < n; i++) y[i] *= v;
}

void orc_flash_attn_ext(const float *q, int64_t qs1, int64_t qs2, int64_t qs3,
                        const float *k, int64_t ks1, int64_t ks2, int64_t ks3,
                        const float *v, int64_t vs1, int64_t vs2, int64_t vs3,
                        int64_t D, int64_t Nq, int64_t Nkv, int64_t nh, int64_t B,
                        float scale, float *o, int nthreads) {
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
    {
        float *VKQ = (float *)malloc((size_t)D * 4);
        float *Vrow = (float *)malloc((size_t)D * 4);
        float *Qrow = (float *)malloc((size_t)D * 4);
#pragma omp for schedule(dynamic, 16)
        for (int64_t r = 0; r < B * nh * Nq; r++) {
            const int64_t b = r / (nh * Nq), h = (r / Nq) % nh, i = r % Nq;
            for (int64_t d = 0; d < D; d++) Qrow[d] = q[b * qs3 + h * qs2 + i * qs1 + d];
            float S = 0.0f, M = -INFINITY;
            memset(VKQ, 0, (size_t)D * 4);
            for (int64_t j = 0; j < Nkv; j++) {
                const float *kr = k + b * ks3 + h * ks2 + j * ks1;
                /* K rows are contiguous in d (unit stride) in every caller. */
                float s = arm_variant() ? vec_dot_f32_neon(D, kr, Qrow) : vec_dot_f32(D, kr, Qrow);
                s = s * scale;
                const float Mold = M;
                float ms = 1.0f, vs = 1.0f;
                if (s > M) {
                    M = s;
                    ms = expf(Mold - M);
                    vec_scale_f32(D, VKQ, ms);
                } else {
                    vs = expf(s - M);
                }
                for (int64_t d = 0; d < D; d++) Vrow[d] = v[b * vs3 + h * vs2 + j * vs1 + d];
                vec_mad_f32(D, VKQ, Vrow, vs);
                S = S * ms + vs;
            }
            const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
            vec_scale_f32(D, VKQ, S_inv);
            memcpy(o + ((b * Nq + i) * nh + h) * D, VKQ, (size_t)D * 4);
        }
        free(VKQ);
        free(Vrow);
        free(Qrow);
    }
}

/* ------------------------------------------------------------------------ */
/* sam3_compute_axial_cis (sam3.cpp:3555-3586). */
void orc_compute_axial_cis(float *out, int dim, int end_x, int end_y, float theta, float scale_pos) {
    const int half_dim = dim / 4;
    float freqs[256];
    for (int i = 0; i < half_dim; ++i) {
        freqs[i] = 1.0f / powf(theta, (float)(i * 4) / (float)dim);
    }
    const int N = end_x * end_y;
    for (int idx = 0; idx < N; ++idx) {
        const float t_x = (float)(idx % end_x) * scale_pos;
        const int row = idx / end_x;
        const float t_y = (float)row * scale_pos;
        for (int i = 0; i < half_dim; ++i) {
            const float ax = t_x * freqs[i];
            out[idx * dim + i * 2 + 0] = cosf(ax);
            out[idx * dim + i * 2 + 1] = sinf(ax);
        }
        for (int i = 0; i < half_dim; ++i) {
            const float ay = t_y * freqs[i];
            out[idx * dim + half_dim * 2 + i * 2 + 0] = cosf(ay);
            out[idx * dim + half_dim * 2 + i * 2 + 1] = sinf(ay);
        }
    }
}

/* sam3_resize_bilinear + sam3_preprocess_image (sam3.cpp:3441-3514). */
/* sam3_resize_bilinear (sam3.cpp:3441-3484): uint8 bilinear, half-pixel
 * centres, double arithmetic, round half up. */
void orc_resize_bilinear_u8(const uint8_t *img, int w, int h, uint8_t *out, int ow, int oh) {
    const double sx = (double)w / ow, sy = (double)h / oh;
    for (int y = 0; y < oh; ++y) {
        double fy = (y + 0.5) * sy - 0.5;
        if (fy < 0.0) fy = 0.0;
        const int y0 = (int)fy;
        const int y1 = (y0 < h - 1) ? y0 + 1 : y0;
        const double wy = fy - y0, wy0 = 1.0 - wy;
        for (int x = 0; x < ow; ++x) {
            double fx = (x + 0.5) * sx - 0.5;
            if (fx < 0.0) fx = 0.0;
            const int x0 = (int)fx;
            const int x1 = (x0 < w - 1) ? x0 + 1 : x0;
            const double wx = fx - x0, wx0 = 1.0 - wx;
            for (int c = 0; c < 3; ++c) {
                const double p00 = img[(y0 * w + x0) * 3 + c], p01 = img[(y0 * w + x1) * 3 + c];
                const double p10 = img[(y1 * w + x0) * 3 + c], p11 = img[(y1 * w + x1) * 3 + c];
                const double vv = wy0 * (wx0 * p00 + wx * p01) + wy * (wx0 * p10 + wx * p11);
                int iv = (int)(vv + 0.5);
                if (iv < 0) iv = 0;
                if (iv > 255) iv = 255;
                out[((size_t)y * ow + x) * 3 + c] = (uint8_t)iv;
            }
        }
    }
}

void orc_preprocess_sam3(const uint8_t *img, int w, int h, int img_size, float *chw) {
    uint8_t *resized = NULL;
    const uint8_t *px = img;
    if (w != img_size || h != img_size) {
        resized = (uint8_t *)malloc((size_t)img_size * img_size * 3);
        orc_resize_bilinear_u8(img, w, h, resized, img_size, img_size);
        px = resized;
    }
    const size_t plane = (size_t)img_size * img_size;
    for (int c = 0; c < 3; ++c) {
        for (int y = 0; y < img_size; ++y) {
            for (int x = 0; x < img_size; ++x) {
                const float vv = px[(y * img_size + x) * 3 + c] / 255.0f;
                chw[c * plane + (size_t)y * img_size + x] = (vv - 0.5f) / 0.5f;
            }
        }
    }
    free(resized);
}
