/*
 * oracle.cpp — CPU restatement of diffuse-cpp's denoising path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
 * CPU baseline.  The product never links, loads or calls this file.
 *
 * Compiled with -ffp-contract=off so every a*b+c rounds twice, as the reference's
 * own files (built for baseline x86-64, no FMA) and GGML's scalar codecs do; the
 * only fused multiply-adds are the explicit fmaf() calls of the block dot products.
 *
 * Parity pins (what fixes each function; the tests live in tests/test_oracle_*.py):
 *   fp16 conversion ........ numpy float16 (IEEE binary16, round-to-nearest-even), all 65536 codes
 *   dequant Q8_0/Q4_K/Q6_K . hand-built blocks with every scale/min/nibble value, checked against
 *                            the closed form y=(d*sc)*q-(dmin*m) written independently in numpy
 *   quantize Q8_K / Q8_0 ... round-trip bound |x - d*q| <= d/2, sign/zero-block special cases
 *   vec_dot ................ exact int64 brute force on dequantised blocks (f64), all types
 *   mul_mat ................ f64 brute force on tiny shapes (dequant W, quantise/dequant X)
 *   rms_norm ............... closed form in f64
 *   rope NEOX .............. position 0 = identity, norm preserved per pair, theta closed form
 *   attention .............. f64 softmax brute force; key-permutation invariance; GQA == MHA
 *                            with repeated KV heads
 *   forward full/cached .... cached == full when the active set is everything; cached with a
 *                            subset == full on positions whose inputs did not change
 *   schedule ............... the integer unmask sequences the cosine/linear formulas give
 *   entropy / top2 ......... uniform row -> ln V, one-hot row -> 0, ties -> lowest index
 *   ordering ............... brute force over the comparator of src/diffuse-sampler.cpp:279-305
 * Parity unpinned against GGML itself: GGML is an empty submodule in the reference
 * (.gitmodules:1-3), so its SIMD float accumulation order, its SIMD expf/silu and its
 * x86 quantize_row_q8_K rounding cannot be run here; the restatement uses the scalar
 * ("generic") forms of those routines.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>
#include <stdlib.h>

#include <algorithm>
#include <numeric>
#include <random>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Block layouts (GGML ggml-common.h; QK_K = 256)                            */
/* ------------------------------------------------------------------------ */
#define QK_K  256
#define QK8_0 32

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[QK8_0]; } blk_q8_0;                         /*  34 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; } blk_q4_K; /* 144 B */
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; } blk_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } blk_q8_K;    /* 292 B */
#pragma pack(pop)

static_assert(sizeof(blk_q8_0) == 34, "q8_0");
static_assert(sizeof(blk_q4_K) == 144, "q4_K");
static_assert(sizeof(blk_q6_K) == 210, "q6_K");
static_assert(sizeof(blk_q8_K) == 292, "q8_K");

/* ------------------------------------------------------------------------ */
/* fp16 (GGML on x86 converts with F16C, round-to-nearest-even)              */
/* ------------------------------------------------------------------------ */
extern "C" float orc_fp16_to_fp32(uint16_t h) { return _cvtsh_ss(h); }
extern "C" uint16_t orc_fp32_to_fp16(float f) { return (uint16_t)_cvtss_sh(f, 0); }
extern "C" void orc_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fp16_to_fp32(x[i]);
}
extern "C" void orc_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fp32_to_fp16(x[i]);
}

extern "C" int64_t orc_block_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: case ORC_TYPE_F16: return 1;
        case ORC_TYPE_Q8_0: return QK8_0;
        case ORC_TYPE_Q4_K: case ORC_TYPE_Q6_K: case ORC_TYPE_Q8_K: return QK_K;
    }
    return 0;
}
extern "C" int64_t orc_type_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: return 4;
        case ORC_TYPE_F16: return 2;
        case ORC_TYPE_Q8_0: return sizeof(blk_q8_0);
        case ORC_TYPE_Q4_K: return sizeof(blk_q4_K);
        case ORC_TYPE_Q6_K: return sizeof(blk_q6_K);
        case ORC_TYPE_Q8_K: return sizeof(blk_q8_K);
    }
    return 0;
}
extern "C" int64_t orc_row_size(int type, int64_t n) {
    int64_t bs = orc_block_size(type);
    if (bs <= 0 || n % bs) return -1;
    return n / bs * orc_type_size(type);
}

/* ------------------------------------------------------------------------ */
/* Dequantisation (GGML dequantize_row_*; scalar forms)                      */
/* ------------------------------------------------------------------------ */
/* 6-bit scale / min of sub-block j of a Q4_K block (GGML get_scale_min_k4). */
static inline void q4k_scale_min(int j, const uint8_t * s, uint8_t * sc, uint8_t * m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m  = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m  = (uint8_t)((s[j + 4] >> 4)   | ((s[j]     >> 6) << 4));
    }
}

static void dequant_q8_0(const blk_q8_0 * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < QK8_0; j++) y[i * QK8_0 + j] = (float)x[i].qs[j] * d;
    }
}

static void dequant_q4_K(const blk_q4_K * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        const float dmin = orc_fp16_to_fp32(x[i].dmin);
        const uint8_t * q = x[i].qs;
        for (int g = 0; g < 4; g++) {            /* 64 elements per group, 2 sub-blocks */
            uint8_t sc, m;
            q4k_scale_min(2 * g, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            q4k_scale_min(2 * g + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; l++) y[l]      = d1 * (float)(q[l] & 0x0F) - m1;
            for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float)(q[l] >> 4)   - m2;
            y += 64;
            q += 32;
        }
    }
}

static inline int q6k_value(const blk_q6_K * b, int e) {
    const int half = e >> 7, r = e & 127, quarter = r >> 5, l = r & 31;
    const uint8_t lo = b->ql[half * 64 + l + (quarter & 1) * 32];
    const int low4 = (quarter < 2) ? (lo & 0x0F) : (lo >> 4);
    const int hi2 = (b->qh[half * 32 + l] >> (2 * quarter)) & 3;
    return (low4 | (hi2 << 4)) - 32;
}

static void dequant_q6_K(const blk_q6_K * x, float * y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int e = 0; e < QK_K; e++) {
            const float ds = d * (float)x[i].scales[e >> 4];   /* scale of 16-element sub-block */
            y[e] = ds * (float)q6k_value(&x[i], e);
        }
        y += QK_K;
    }
}

extern "C" int orc_dequant_row(int type, const void * x, float * y, int64_t n) {
    const int64_t bs = orc_block_size(type);
    if (bs <= 0 || n % bs) return -1;
    switch (type) {
        case ORC_TYPE_F32: memcpy(y, x, (size_t)n * 4); return 0;
        case ORC_TYPE_F16: orc_fp16_to_fp32_row((const uint16_t *)x, y, n); return 0;
        case ORC_TYPE_Q8_0: dequant_q8_0((const blk_q8_0 *)x, y, n / bs); return 0;
        case ORC_TYPE_Q4_K: dequant_q4_K((const blk_q4_K *)x, y, n / bs); return 0;
        case ORC_TYPE_Q6_K: dequant_q6_K((const blk_q6_K *)x, y, n / bs); return 0;
        case ORC_TYPE_Q8_K: {
            const blk_q8_K * b = (const blk_q8_K *)x;
            for (int64_t i = 0; i < n / bs; i++)
                for (int j = 0; j < QK_K; j++) y[i * QK_K + j] = b[i].d * (float)b[i].qs[j];
            return 0;
        }
    }
    return -1;
}

/* ------------------------------------------------------------------------ */
/* Activation quantisation (GGML quantize_row_q8_K_ref / quantize_row_q8_0_ref) */
/* ------------------------------------------------------------------------ */
/* Round half to even via the 1.5*2^23 trick (GGML nearest_int). */
static inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

extern "C" void orc_quantize_row_q8_K(const float * x, void * vy, int64_t k) {
    blk_q8_K * y = (blk_q8_K *)vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        if (amax == 0.0f) {
            y[i].d = 0;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            x += QK_K;
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; j++) {
            const int v = nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[j * 16 + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1 / iscale;
        x += QK_K;
    }
}

extern "C" void orc_quantize_row_q8_0(const float * x, void * vy, int64_t k) {
    blk_q8_0 * y = (blk_q8_0 *)vy;
    const int64_t nb = k / QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = orc_fp32_to_fp16(d);
        for (int j = 0; j < QK8_0; j++) y[i].qs[j] = (int8_t)roundf(x[i * QK8_0 + j] * id);
    }
}

/* ------------------------------------------------------------------------ */
/* vec_dot (GGML ggml_vec_dot_*_generic: integer block sums, float scale per */
/* block; float accumulation order across blocks is unpinned)               */
/* ------------------------------------------------------------------------ */
/* Integer parts of the block dots.  The AVX2 forms compute the same integers as the
 * scalar definitions (u8 x s8 pair sums fit int16 without saturation: 2*63*127). */
static inline int32_t hsum_i32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

/* isum = sum_j sc_j * sum_{l<32} q4[32j+l] * q8[32j+l] over one Q4_K super-block */
static inline int32_t q4k_isum(const uint8_t * qs, const int8_t * q8, const uint8_t sc[8]) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256i acc = _mm256_setzero_si256();
    for (int g = 0; g < 4; g++) {
        const __m256i q4 = _mm256_loadu_si256((const __m256i *)(qs + 32 * g));
        const __m256i lo = _mm256_and_si256(q4, m4);
        const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4);
        const __m256i p0 = _mm256_maddubs_epi16(lo, _mm256_loadu_si256((const __m256i *)(q8 + 64 * g)));
        const __m256i p1 = _mm256_maddubs_epi16(hi, _mm256_loadu_si256((const __m256i *)(q8 + 64 * g + 32)));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p0, _mm256_set1_epi16(sc[2 * g])));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p1, _mm256_set1_epi16(sc[2 * g + 1])));
    }
    return hsum_i32(acc);
}

/* sum_j sc_j * sum_{l<16} u6[16j+l] * q8[16j+l] with u6 = q + 32 in [0, 63] */
static inline int32_t q6k_usum(const uint8_t * u6, const int8_t * q8, const int8_t * sc) {
    __m256i acc = _mm256_setzero_si256();
    for (int j = 0; j < 16; j += 2) {
        const __m256i p = _mm256_maddubs_epi16(_mm256_loadu_si256((const __m256i *)(u6 + 16 * j)),
                                               _mm256_loadu_si256((const __m256i *)(q8 + 16 * j)));
        const __m256i s = _mm256_setr_epi16(sc[j], sc[j], sc[j], sc[j], sc[j], sc[j], sc[j], sc[j], sc[j + 1],
                                            sc[j + 1], sc[j + 1], sc[j + 1], sc[j + 1], sc[j + 1], sc[j + 1], sc[j + 1]);
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p, s));
    }
    return hsum_i32(acc);
}

/* sum_{l<32} a[l] * b[l], both int8 */
static inline int32_t i8_dot32(const int8_t * a, const int8_t * b) {
    const __m256i va = _mm256_loadu_si256((const __m256i *)a), vb = _mm256_loadu_si256((const __m256i *)b);
    const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(va, va), _mm256_sign_epi8(vb, va));
    return hsum_i32(_mm256_madd_epi16(p, _mm256_set1_epi16(1)));
}

/* Block dot products.  Integer parts are GGML's (exact int32 sums); the float part
 * folds the block scales in a fixed order that the GPU kernels reproduce bit for bit:
 *   Q4_K  x = d_w*isum;  x = fma(-dmin_w, msum, x);  S = fma(d_a, x, S)
 *   Q6_K  x = d_w*isum;  S = fma(d_a, x, S)
 *   Q8_0  x = d_w*isum;  S = fma(d_a, x, S)         (per 32-element block)
 * The K range is cut into chunks of ORC_DOT_CHUNK elements: S restarts at 0 in every
 * chunk and the chunk sums are added in order, T = T + S (T starts at 0).  GGML folds
 * the same factors as (d_w*d_a)*isum, in float, in its own SIMD lane order; the value
 * is the same up to float rounding. */
#define ORC_DOT_CHUNK 2048
static float dot_q4_K_q8_K(int64_t n, const blk_q4_K * x, const blk_q8_K * y) {
    float T = 0.0f, S = 0.0f;
    const int64_t per = ORC_DOT_CHUNK / QK_K;
    for (int64_t i = 0; i < n / QK_K; i++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) q4k_scale_min(j, x[i].scales, &sc[j], &mn[j]);
        const int32_t isum = q4k_isum(x[i].qs, y[i].qs, sc);
        int32_t msum = 0;
        for (int j = 0; j < 8; j++)
            msum += (int32_t)mn[j] * ((int32_t)y[i].bsums[2 * j] + (int32_t)y[i].bsums[2 * j + 1]);
        const float dw = orc_fp16_to_fp32(x[i].d), dmw = orc_fp16_to_fp32(x[i].dmin);
        float t = dw * (float)isum;
        t = fmaf(-dmw, (float)msum, t);
        S = fmaf(y[i].d, t, S);
        if ((i + 1) % per == 0 || i + 1 == n / QK_K) { T = T + S; S = 0.0f; }
    }
    return T;
}

static float dot_q6_K_q8_K(int64_t n, const blk_q6_K * x, const blk_q8_K * y) {
    float T = 0.0f, sum = 0.0f;
    const int64_t per = ORC_DOT_CHUNK / QK_K;
    uint8_t u6[QK_K];
    for (int64_t i = 0; i < n / QK_K; i++) {
        /* unpack q + 32 (ql low/high nibbles and qh 2-bit fields, GGML block_q6_K order) */
        for (int half = 0; half < 2; half++) {
            const uint8_t * ql = x[i].ql + 64 * half;
            const uint8_t * qh = x[i].qh + 32 * half;
            uint8_t * u = u6 + 128 * half;
            for (int l = 0; l < 32; l++) {
                u[l]      = (uint8_t)((ql[l] & 0x0F)      | (((qh[l] >> 0) & 3) << 4));
                u[l + 32] = (uint8_t)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4));
                u[l + 64] = (uint8_t)((ql[l] >> 4)        | (((qh[l] >> 4) & 3) << 4));
                u[l + 96] = (uint8_t)((ql[l + 32] >> 4)   | (((qh[l] >> 6) & 3) << 4));
            }
        }
        /* isum = sum_j sc_j * sum_l (u6 - 32) * q8 */
        int32_t corr = 0;
        for (int j = 0; j < 16; j++) corr += (int32_t)x[i].scales[j] * (int32_t)y[i].bsums[j];
        const int32_t isum = q6k_usum(u6, y[i].qs, x[i].scales) - 32 * corr;
        const float t = orc_fp16_to_fp32(x[i].d) * (float)isum;
        sum = fmaf(y[i].d, t, sum);
        if ((i + 1) % per == 0 || i + 1 == n / QK_K) { T = T + sum; sum = 0.0f; }
    }
    return T;
}

static float dot_q8_0_q8_0(int64_t n, const blk_q8_0 * x, const blk_q8_0 * y) {
    float T = 0.0f, sum = 0.0f;
    const int64_t per = ORC_DOT_CHUNK / QK8_0;
    for (int64_t i = 0; i < n / QK8_0; i++) {
        const int32_t s = i8_dot32(x[i].qs, y[i].qs);
        const float t = orc_fp16_to_fp32(x[i].d) * (float)s;
        sum = fmaf(orc_fp16_to_fp32(y[i].d), t, sum);
        if ((i + 1) % per == 0 || i + 1 == n / QK8_0) { T = T + sum; sum = 0.0f; }
    }
    return T;
}

/* F16 / F32 dots: f32 products (rounded to float, as GGML's scalar ggml_vec_dot_f16 /
 * ggml_vec_dot_f32 form them) summed in double (ggml_float), in 16 interleaved lanes
 * (lane l takes elements l, l+16, ...; the lanes are added in order at the end).  The
 * lane order is this restatement's own (GGML's SIMD paths sum in float lanes of their own). */
/* lanes added in order, then the tail (elements past the last whole 16) */
static inline float dot_lanes_end(__m256d a0, __m256d a1, __m256d a2, __m256d a3, double tail) {
    alignas(32) double v[16];
    _mm256_store_pd(v, a0);
    _mm256_store_pd(v + 4, a1);
    _mm256_store_pd(v + 8, a2);
    _mm256_store_pd(v + 12, a3);
    double s = 0.0;
    for (int l = 0; l < 16; l++) s += v[l];
    return (float)(s + tail);
}

static float dot_f16_f16(int64_t n, const uint16_t * x, const uint16_t * y) {
    __m256d a0 = _mm256_setzero_pd(), a1 = a0, a2 = a0, a3 = a0;
    int64_t i = 0;
    for (; i + 16 <= n; i += 16) {
        const __m256 p0 = _mm256_mul_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x + i))),
                                        _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i))));
        const __m256 p1 = _mm256_mul_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x + i + 8))),
                                        _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i + 8))));
        a0 = _mm256_add_pd(a0, _mm256_cvtps_pd(_mm256_castps256_ps128(p0)));
        a1 = _mm256_add_pd(a1, _mm256_cvtps_pd(_mm256_extractf128_ps(p0, 1)));
        a2 = _mm256_add_pd(a2, _mm256_cvtps_pd(_mm256_castps256_ps128(p1)));
        a3 = _mm256_add_pd(a3, _mm256_cvtps_pd(_mm256_extractf128_ps(p1, 1)));
    }
    double t = 0.0;
    for (; i < n; i++) t += (double)(orc_fp16_to_fp32(x[i]) * orc_fp16_to_fp32(y[i]));
    return dot_lanes_end(a0, a1, a2, a3, t);
}

static float dot_f32(int64_t n, const float * x, const float * y) {
    __m256d a0 = _mm256_setzero_pd(), a1 = a0, a2 = a0, a3 = a0;
    int64_t i = 0;
    for (; i + 16 <= n; i += 16) {
        const __m256 p0 = _mm256_mul_ps(_mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i));
        const __m256 p1 = _mm256_mul_ps(_mm256_loadu_ps(x + i + 8), _mm256_loadu_ps(y + i + 8));
        a0 = _mm256_add_pd(a0, _mm256_cvtps_pd(_mm256_castps256_ps128(p0)));
        a1 = _mm256_add_pd(a1, _mm256_cvtps_pd(_mm256_extractf128_ps(p0, 1)));
        a2 = _mm256_add_pd(a2, _mm256_cvtps_pd(_mm256_castps256_ps128(p1)));
        a3 = _mm256_add_pd(a3, _mm256_cvtps_pd(_mm256_extractf128_ps(p1, 1)));
    }
    double t = 0.0;
    for (; i < n; i++) t += (double)(x[i] * y[i]);
    return dot_lanes_end(a0, a1, a2, a3, t);
}

/* Attention dot products: f32 x f32 products are exact in f64 and are summed in f64,
 * then rounded once, so the float result does not depend on the summation order
 * (the CPU path accumulates in its own SIMD order; the value it approximates is this). */
static float dot_f32_exact(int64_t n, const float * x, const float * y) {
    double s = 0.0;
    for (int64_t i = 0; i < n; i++) s += (double)x[i] * (double)y[i];
    return (float)s;
}

/* vec_dot_type of each weight type, and the byte size of one converted row. */
static int vec_dot_type(int wtype) {
    switch (wtype) {
        case ORC_TYPE_Q4_K: case ORC_TYPE_Q6_K: return ORC_TYPE_Q8_K;
        case ORC_TYPE_Q8_0: return ORC_TYPE_Q8_0;
        case ORC_TYPE_F16: return ORC_TYPE_F16;
        case ORC_TYPE_F32: return ORC_TYPE_F32;
    }
    return -1;
}

static void convert_act_row(int vdt, const float * x, void * out, int64_t k) {
    switch (vdt) {
        case ORC_TYPE_Q8_K: orc_quantize_row_q8_K(x, out, k); break;
        case ORC_TYPE_Q8_0: orc_quantize_row_q8_0(x, out, k); break;
        case ORC_TYPE_F16:  orc_fp32_to_fp16_row(x, (uint16_t *)out, k); break;
        case ORC_TYPE_F32:  memcpy(out, x, (size_t)k * 4); break;
    }
}

static float vec_dot_any(int wtype, int64_t n, const void * w, const void * a) {
    switch (wtype) {
        case ORC_TYPE_Q4_K: return dot_q4_K_q8_K(n, (const blk_q4_K *)w, (const blk_q8_K *)a);
        case ORC_TYPE_Q6_K: return dot_q6_K_q8_K(n, (const blk_q6_K *)w, (const blk_q8_K *)a);
        case ORC_TYPE_Q8_0: return dot_q8_0_q8_0(n, (const blk_q8_0 *)w, (const blk_q8_0 *)a);
        case ORC_TYPE_F16:  return dot_f16_f16(n, (const uint16_t *)w, (const uint16_t *)a);
        case ORC_TYPE_F32:  return dot_f32(n, (const float *)w, (const float *)a);
    }
    return NAN;
}

extern "C" int orc_vec_dot(int wtype, int64_t n, const void * w_row, const void * a_row, float * out) {
    if (vec_dot_type(wtype) < 0 || orc_row_size(wtype, n) < 0) return -1;
    *out = vec_dot_any(wtype, n, w_row, a_row);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* mul_mat (GGML ggml_compute_forward_mul_mat: src1 -> vec_dot_type, then    */
/* one vec_dot per output element); called at src/diffuse-graph.cpp:61-63,   */
/* 122, 136-140, 154 and the cached twins 451-453, 556, 570-574, 587         */
/* ------------------------------------------------------------------------ */
extern "C" int orc_mul_mat(int wtype, const void * W, int64_t N, int64_t K,
                           const float * X, int64_t M, float * Y, int n_threads) {
    const int vdt = vec_dot_type(wtype);
    const int64_t wrow = orc_row_size(wtype, K), arow = orc_row_size(vdt, K);
    if (vdt < 0 || wrow < 0 || arow < 0) return -1;
    std::vector<uint8_t> act((size_t)(arow * M));
    #pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t m = 0; m < M; m++) convert_act_row(vdt, X + m * K, act.data() + m * arow, K);

    #pragma omp parallel for num_threads(n_threads) schedule(dynamic, 8)
    for (int64_t n = 0; n < N; n++) {
        const uint8_t * w = (const uint8_t *)W + n * wrow;
        for (int64_t m = 0; m < M; m++) Y[m * N + n] = vec_dot_any(wtype, K, w, act.data() + m * arow);
    }
    return 0;
}

/* rms_norm then ggml_mul by the (F32-cast) norm weight
 * (src/diffuse-graph.cpp:51-58; GGML ggml_compute_forward_rms_norm_f32:
 *  sum of float squares accumulated in double, scale = 1/sqrtf(mean + eps)). */
extern "C" void orc_rms_norm_mul(const float * x, const float * w, int64_t M, int64_t K, float eps, float * y) {
    for (int64_t m = 0; m < M; m++) {
        const float * xr = x + m * K;
        double sum = 0.0;
        for (int64_t k = 0; k < K; k++) sum += (double)(xr[k] * xr[k]);
        const float mean = (float)(sum / (double)K);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t k = 0; k < K; k++) y[m * K + k] = (xr[k] * scale) * w[k];
    }
}

/* NEOX rope angles (GGML ggml_rope_cache_init with freq_scale=1, ext_factor=0,
 * attn_factor=1): theta_0 = p, theta_{i+1} = theta_i * powf(base, -2/n_dims),
 * cos/sin by cosf/sinf.  Used at src/diffuse-graph.cpp:76-79 and 466-469. */
extern "C" void orc_rope_table(int n_pos, int head_dim, float theta_base, float * tab) {
    const int half = head_dim / 2;
    const float theta_scale = powf(theta_base, -2.0f / (float)head_dim);
    for (int p = 0; p < n_pos; p++) {
        float theta = (float)p;
        for (int i = 0; i < half; i++) {
            tab[((size_t)p * half + i) * 2 + 0] = cosf(theta);
            tab[((size_t)p * half + i) * 2 + 1] = sinf(theta);
            theta *= theta_scale;
        }
    }
}

/* x: [M][n_heads][head_dim]; rotate pairs (i, i+half) of each head by pos[m]. */
extern "C" void orc_rope_neox(float * x, int64_t M, int n_heads, int head_dim, const int32_t * pos,
                              const float * tab) {
    const int half = head_dim / 2;
    for (int64_t m = 0; m < M; m++) {
        const float * t = tab + (size_t)pos[m] * half * 2;
        for (int h = 0; h < n_heads; h++) {
            float * v = x + ((size_t)m * n_heads + h) * head_dim;
            for (int i = 0; i < half; i++) {
                const float c = t[2 * i], s = t[2 * i + 1];
                const float x0 = v[i], x1 = v[i + half];
                v[i]        = x0 * c - x1 * s;
                v[i + half] = x0 * s + x1 * c;
            }
        }
    }
}

/* exp inside GGML ops (silu, soft_max) is GGML's own SIMD approximation, which cannot be
 * run here; the restatement uses the correctly rounded expf, (float)exp((double)x). */
static inline float exp_cr(float x) { return (float)exp((double)x); }

extern "C" float orc_silu(float x) { return x / (1.0f + exp_cr(-x)); }

/* ------------------------------------------------------------------------ */
/* Forward pass                                                               */
/* ------------------------------------------------------------------------ */
static std::vector<float> to_f32(const orc_tensor & t) {
    std::vector<float> v((size_t)(t.ne0 * t.ne1));
    if (t.data) {
        const int64_t rs = orc_row_size(t.type, t.ne0);
        for (int64_t r = 0; r < t.ne1; r++)
            orc_dequant_row(t.type, (const uint8_t *)t.data + r * rs, v.data() + r * t.ne0, t.ne0);
    }
    return v;
}

static void add_bias(std::vector<float> & y, int64_t M, int64_t N, const orc_tensor & b) {
    if (!b.data) return;
    std::vector<float> bf = to_f32(b);   /* ensure_f32 (src/diffuse-graph.cpp:4-8) */
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) y[m * N + n] = y[m * N + n] + bf[n];
}

static void embed(const orc_model * md, const int32_t * tok, int M, float * x) {
    const int64_t d = md->n_embd;
    const int64_t rs = orc_row_size(md->tok_embd.type, d);
    for (int m = 0; m < M; m++)
        orc_dequant_row(md->tok_embd.type, (const uint8_t *)md->tok_embd.data + (int64_t)tok[m] * rs, x + m * d, d);
}

/* Attention of M queries over n_keys keys (src/diffuse-graph.cpp:97-119, 528-553):
 * s = dot(K_n, Q_m) * (1/sqrtf(hd)); softmax over the visible keys (max, expf, double
 * sum, multiply by 1/sum); out = sum_n V_n * p_n.  q: [M][H][hd]; k, v: [n_keys][H][hd]
 * (already GQA-expanded); out: [M][H*hd].  Every key is visible unless vis != NULL:
 * then key n is visible to query m when vis->kpos[n] <= vis->qpos[m] and, with a
 * window w > 0, vis->qpos[m] - vis->kpos[n] < w — the causal mask of
 * src/ar-graph.cpp:70-88, whose -inf entries GGML's flash attention skips.  Visible
 * keys are summed in increasing n. */
struct key_vis { const int32_t * qpos; const int32_t * kpos; int window; };

static void attention(const float * q, const float * k, const float * v, int M, int n_keys,
                      int H, int hd, float * out, int n_threads, const key_vis * vis = nullptr) {
    const float scale = 1.0f / sqrtf((float)hd);
    #pragma omp parallel for num_threads(n_threads) collapse(2) schedule(static)
    for (int h = 0; h < H; h++) {
        for (int m = 0; m < M; m++) {
            std::vector<float> s(n_keys);
            std::vector<char> on(n_keys, 1);
            if (vis)
                for (int n = 0; n < n_keys; n++)
                    on[n] = vis->kpos[n] <= vis->qpos[m] && (vis->window <= 0 || vis->qpos[m] - vis->kpos[n] < vis->window);
            const float * qm = q + ((size_t)m * H + h) * hd;
            float mx = -INFINITY;
            for (int n = 0; n < n_keys; n++) {
                if (!on[n]) continue;
                s[n] = dot_f32_exact(hd, k + ((size_t)n * H + h) * hd, qm) * scale;
                mx = fmaxf(mx, s[n]);
            }
            double sum = 0.0;
            for (int n = 0; n < n_keys; n++) {
                if (!on[n]) continue;
                s[n] = exp_cr(s[n] - mx);
                sum += (double)s[n];
            }
            const float inv = (float)(1.0 / sum);
            for (int n = 0; n < n_keys; n++) s[n] = on[n] ? s[n] * inv : 0.0f;
            float * o = out + (size_t)m * H * hd + (size_t)h * hd;
            for (int dd = 0; dd < hd; dd++) {
                double acc = 0.0;
                for (int n = 0; n < n_keys; n++)
                    if (on[n]) acc += (double)v[((size_t)n * H + h) * hd + dd] * (double)s[n];
                o[dd] = (float)acc;
            }
        }
    }
}

extern "C" void orc_attention(const float * q, const float * k, const float * v, int M, int n_keys, int H, int hd,
                              float * out, int n_threads) {
    attention(q, k, v, M, n_keys, H, hd, out, n_threads);
}

extern "C" void orc_attention_causal(const float * q, const float * k, const float * v, int M, int n_keys, int H,
                                     int hd, const int32_t * qpos, const int32_t * kpos, int window, float * out,
                                     int n_threads) {
    const key_vis vis = {qpos, kpos, window};
    attention(q, k, v, M, n_keys, H, hd, out, n_threads, &vis);
}

/* GQA repeat (src/diffuse-graph.cpp:84-95): query head h reads KV head h / n_rep. */
static void expand_heads(const float * src, int M, int Hkv, int H, int hd, float * dst) {
    const int n_rep = H / Hkv;
    for (int m = 0; m < M; m++)
        for (int h = 0; h < H; h++)
            memcpy(dst + ((size_t)m * H + h) * hd, src + ((size_t)m * Hkv + h / n_rep) * hd, (size_t)hd * 4);
}

/* Options of the autoregressive graph (src/ar-graph.cpp:27-196): causal mask with an
 * optional sliding window, skipped layers, and the layer-impact profile. */
struct pass_opts {
    bool            causal = false;
    int             window = 0;
    const uint8_t * skip = nullptr;     /* [n_layer] nonzero = layer left out */
    float *         impact = nullptr;   /* [n_layer] sum of squared layer deltas */
    int             head_from = 0;      /* logits for rows head_from..M-1 only */
};

/* One transformer stack over M rows with RoPE positions pos[].  Keys/values for
 * attention: if kv_cached != NULL, K_full = [gathered cached rows ‖ this pass's rows]
 * (src/diffuse-graph.cpp:497-525); else just this pass's rows.  The per-layer
 * K/V of this pass (after RoPE + GQA expansion) are returned in k_out/v_out. */
static int run_layers(const orc_model * md, const int32_t * tok, const int32_t * pos, int M,
                      const orc_kv * kv_cached, const int32_t * cached_pos, int n_cached,
                      float * logits, float * k_out, float * v_out, int n_threads,
                      const pass_opts & opt = pass_opts()) {
    const int d = md->n_embd, H = md->n_head, Hkv = md->n_head_kv, hd = d / H;
    const int dkv = Hkv * hd, F = md->n_ff, L = md->n_layer;
    const float eps = md->rms_norm_eps;
    int max_pos = 0;
    for (int m = 0; m < M; m++) max_pos = std::max(max_pos, (int)pos[m]);
    std::vector<float> tab((size_t)(max_pos + 1) * hd);
    orc_rope_table(max_pos + 1, hd, md->rope_theta, tab.data());

    std::vector<float> x((size_t)M * d), h((size_t)M * d), q((size_t)M * d), k((size_t)M * dkv),
        v((size_t)M * dkv), ke((size_t)M * d), ve((size_t)M * d), att((size_t)M * d), o((size_t)M * d),
        g((size_t)M * F), u((size_t)M * F);
    const int n_keys = n_cached + M;
    std::vector<float> kf((size_t)n_keys * d), vf((size_t)n_keys * d);
    std::vector<int32_t> kpos(n_keys);
    for (int c = 0; c < n_cached; c++) kpos[c] = cached_pos[c];
    for (int m = 0; m < M; m++) kpos[n_cached + m] = pos[m];
    const key_vis vis = {pos, kpos.data(), opt.window};
    std::vector<float> x_in;
    embed(md, tok, M, x.data());

    for (int il = 0; il < L; il++) {
        if (opt.skip && opt.skip[il]) continue;   /* src/ar-graph.cpp:98-102 */
        if (opt.impact) x_in = x;
        const orc_layer & ly = md->layers[il];
        std::vector<float> w = to_f32(ly.attn_norm);
        orc_rms_norm_mul(x.data(), w.data(), M, d, eps, h.data());
        if (orc_mul_mat(ly.wq.type, ly.wq.data, d, d, h.data(), M, q.data(), n_threads)) return -1;
        if (orc_mul_mat(ly.wk.type, ly.wk.data, dkv, d, h.data(), M, k.data(), n_threads)) return -1;
        if (orc_mul_mat(ly.wv.type, ly.wv.data, dkv, d, h.data(), M, v.data(), n_threads)) return -1;
        add_bias(q, M, d, ly.bq);
        add_bias(k, M, dkv, ly.bk);
        add_bias(v, M, dkv, ly.bv);
        orc_rope_neox(q.data(), M, H, hd, pos, tab.data());
        orc_rope_neox(k.data(), M, Hkv, hd, pos, tab.data());
        expand_heads(k.data(), M, Hkv, H, hd, ke.data());
        expand_heads(v.data(), M, Hkv, H, hd, ve.data());
        if (k_out) {
            memcpy(k_out + (size_t)il * M * d, ke.data(), (size_t)M * d * 4);
            memcpy(v_out + (size_t)il * M * d, ve.data(), (size_t)M * d * 4);
        }
        const float * kk = ke.data();
        const float * vv = ve.data();
        if (kv_cached) {
            const float * kc = kv_cached->k + (size_t)il * kv_cached->n_tokens * d;
            const float * vc = kv_cached->v + (size_t)il * kv_cached->n_tokens * d;
            for (int c = 0; c < n_cached; c++) {
                memcpy(kf.data() + (size_t)c * d, kc + (size_t)cached_pos[c] * d, (size_t)d * 4);
                memcpy(vf.data() + (size_t)c * d, vc + (size_t)cached_pos[c] * d, (size_t)d * 4);
            }
            memcpy(kf.data() + (size_t)n_cached * d, ke.data(), (size_t)M * d * 4);
            memcpy(vf.data() + (size_t)n_cached * d, ve.data(), (size_t)M * d * 4);
            kk = kf.data();
            vv = vf.data();
        }
        attention(q.data(), kk, vv, M, n_keys, H, hd, att.data(), n_threads, opt.causal ? &vis : nullptr);
        if (orc_mul_mat(ly.wo.type, ly.wo.data, d, d, att.data(), M, o.data(), n_threads)) return -1;
        for (size_t i = 0; i < x.size(); i++) x[i] = o[i] + x[i];

        w = to_f32(ly.ffn_norm);
        orc_rms_norm_mul(x.data(), w.data(), M, d, eps, h.data());
        if (orc_mul_mat(ly.ffn_gate.type, ly.ffn_gate.data, F, d, h.data(), M, g.data(), n_threads)) return -1;
        if (orc_mul_mat(ly.ffn_up.type, ly.ffn_up.data, F, d, h.data(), M, u.data(), n_threads)) return -1;
        for (size_t i = 0; i < g.size(); i++) g[i] = orc_silu(g[i]) * u[i];
        if (orc_mul_mat(ly.ffn_down.type, ly.ffn_down.data, d, F, g.data(), M, o.data(), n_threads)) return -1;
        for (size_t i = 0; i < x.size(); i++) x[i] = o[i] + x[i];
        if (opt.impact) {
            /* ggml_sum(ggml_sqr(ggml_sub(out, in))) (src/ar-graph.cpp:219-228): float
             * differences and squares, each row summed in double, rows added in double */
            double tot = 0.0;
            for (int m = 0; m < M; m++) {
                double rs = 0.0;
                for (int i = 0; i < d; i++) {
                    const float df = x[(size_t)m * d + i] - x_in[(size_t)m * d + i];
                    rs += (double)(df * df);
                }
                tot += rs;
            }
            opt.impact[il] = (float)tot;
        }
    }
    std::vector<float> w = to_f32(md->output_norm);
    const int hf = opt.head_from;
    orc_rms_norm_mul(x.data() + (size_t)hf * d, w.data(), M - hf, d, eps, h.data());
    return orc_mul_mat(md->output.type, md->output.data, md->n_vocab, d, h.data(), M - hf, logits, n_threads);
}

extern "C" int orc_forward_full(const orc_model * md, const int32_t * tokens, int n, float * logits,
                                orc_kv * kv, int n_threads) {
    std::vector<int32_t> pos(n);
    std::iota(pos.begin(), pos.end(), 0);
    if (!kv) return run_layers(md, tokens, pos.data(), n, nullptr, nullptr, 0, logits, nullptr, nullptr, n_threads);
    /* K/V of all positions go straight to the cache (src/diffuse-graph.cpp:356-375). */
    const size_t per = (size_t)n * md->n_embd;
    std::vector<float> ko(per * md->n_layer), vo(per * md->n_layer);
    int rc = run_layers(md, tokens, pos.data(), n, nullptr, nullptr, 0, logits, ko.data(), vo.data(), n_threads);
    if (rc) return rc;
    const size_t cap = (size_t)kv->n_tokens * md->n_embd;
    for (uint32_t il = 0; il < md->n_layer; il++) {
        memcpy(kv->k + il * cap, ko.data() + il * per, per * 4);
        memcpy(kv->v + il * cap, vo.data() + il * per, per * 4);
    }
    return 0;
}

extern "C" int orc_forward_cached(const orc_model * md, const int32_t * active_tokens,
                                  const int32_t * active_pos, int n_active, int n_total, orc_kv * kv,
                                  const int32_t * cached_pos, float * logits, int n_threads) {
    const int n_cached = n_total - n_active;
    const size_t per = (size_t)n_active * md->n_embd;
    std::vector<float> ko(per * md->n_layer), vo(per * md->n_layer);
    int rc = run_layers(md, active_tokens, active_pos, n_active, kv, cached_pos, n_cached, logits,
                        ko.data(), vo.data(), n_threads);
    if (rc) return rc;
    /* update_kv scatter (src/diffuse-cache.h:124-140) */
    const size_t cap = (size_t)kv->n_tokens * md->n_embd;
    for (uint32_t il = 0; il < md->n_layer; il++)
        for (int a = 0; a < n_active; a++) {
            memcpy(kv->k + il * cap + (size_t)active_pos[a] * md->n_embd, ko.data() + il * per + (size_t)a * md->n_embd, md->n_embd * 4);
            memcpy(kv->v + il * cap + (size_t)active_pos[a] * md->n_embd, vo.data() + il * per + (size_t)a * md->n_embd, md->n_embd * 4);
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Sampler (src/diffuse-sampler.cpp)                                          */
/* ------------------------------------------------------------------------ */
/* src/diffuse-sampler.cpp:12-31 */
extern "C" int orc_tokens_to_unmask(int step, int total_steps, int total_masked, int schedule) {
    const float t0 = (float)step / total_steps;
    const float t1 = (float)(step + 1) / total_steps;
    float frac;
    if (schedule == ORC_SCHED_COSINE) {
        /* t * M_PI is evaluated in double, then narrowed for cosf, as in the reference */
        const float c0 = cosf(t0 * M_PI * 0.5f);
        const float c1 = cosf(t1 * M_PI * 0.5f);
        frac = (c0 - c1) / c0;
    } else {
        frac = 1.0f / (float)(total_steps - step);
    }
    int n = (int)roundf(frac * (float)total_masked);
    if (n < 1 && total_masked > 0) n = 1;
    return std::min(n, total_masked);
}

/* src/diffuse-sampler.cpp:34-57 */
extern "C" float orc_entropy(const float * x, int V) {
    float mx = x[0];
    for (int v = 1; v < V; v++) if (x[v] > mx) mx = x[v];
    float sum = 0.0f;
    for (int v = 0; v < V; v++) sum += expf(x[v] - mx);
    const float log_sum = logf(sum);
    float ent = 0.0f;
    for (int v = 0; v < V; v++) {
        const float lp = (x[v] - mx) - log_sum;
        const float p = expf(lp);
        if (p > 1e-10f) ent -= p * lp;
    }
    return ent;
}

/* src/diffuse-sampler.cpp:241-252 */
extern "C" void orc_top2(const float * x, int V, int * best, float * best_val, float * second_val) {
    int b = 0;
    float bv = x[0], sv = -1e30f;
    for (int v = 1; v < V; v++) {
        if (x[v] > bv) { sv = bv; bv = x[v]; b = v; }
        else if (x[v] > sv) { sv = x[v]; }
    }
    *best = b; *best_val = bv; *second_val = sv;
}

/* src/diffuse-sampler.cpp:277-305 with ties broken by position ascending. */
extern "C" int orc_order_candidates(orc_candidate * c, int n, int remasking, float tau, int n_sched) {
    if (remasking == ORC_REMASK_ENTROPY_EXIT) {
        std::sort(c, c + n, [](const orc_candidate & a, const orc_candidate & b) {
            if (a.entropy != b.entropy) return a.entropy < b.entropy;
            return a.pos < b.pos;
        });
        int n_easy = 0;
        for (int i = 0; i < n; i++) { if (c[i].entropy < tau) n_easy++; else break; }
        return std::min(std::max(n_sched, n_easy), n);
    }
    if (remasking == ORC_REMASK_LOW_CONFIDENCE || remasking == ORC_REMASK_MASKGIT_PLUS ||
        remasking == ORC_REMASK_TOPK_MARGIN) {
        std::sort(c, c + n, [](const orc_candidate & a, const orc_candidate & b) {
            if (a.confidence != b.confidence) return a.confidence > b.confidence;
            return a.pos < b.pos;
        });
    }
    return std::min(n_sched, n);
}

/* diffuse_sample (src/diffuse-sampler.cpp:60-370) with its cache (src/diffuse-cache.h). */
extern "C" int orc_generate(const orc_model * md, const int32_t * prompt, int n_prompt, int n_generate,
                            const orc_sampler_params * p, int32_t * out, orc_gen_stats * stats,
                            int n_threads) {
    const int V = md->n_vocab, mask_id = md->mask_token_id, d = md->n_embd;
    const bool shift = md->is_dream != 0;
    const int N = n_prompt + n_generate;
    std::vector<int32_t> seq(prompt, prompt + n_prompt);
    seq.resize(N, mask_id);
    std::vector<bool> is_masked(N, false);
    for (int i = n_prompt; i < N; i++) is_masked[i] = true;
    int n_masked = n_generate;
    std::vector<float> logits_full((size_t)N * V);
    std::mt19937 rng(p->seed);

    const bool use_cache = p->use_cache != 0;
    std::vector<float> kc, vc;
    orc_kv kv = {N, nullptr, nullptr};
    std::vector<int32_t> prev_seq(N, -1);
    std::vector<int> last_changed(N, -1);
    bool cache_init = false;
    if (use_cache) {
        kc.assign((size_t)md->n_layer * N * d, 0.0f);
        vc.assign((size_t)md->n_layer * N * d, 0.0f);
        kv.k = kc.data();
        kv.v = vc.data();
    }
    if (stats) memset(stats, 0, sizeof(*stats));

    for (int step = 0; step < p->n_steps && n_masked > 0; step++) {
        int rows = N;
        const bool force_full = !use_cache || !cache_init ||
                                (p->cache_refresh > 0 && step > 0 && step % p->cache_refresh == 0);
        bool full = force_full;
        std::vector<int32_t> act, cached;
        if (!force_full) {
            /* compute_active_set (src/diffuse-cache.h:79-116) */
            for (int i = 0; i < N; i++) {
                const bool changed = seq[i] != prev_seq[i];
                if (changed) last_changed[i] = step;
                const bool recent = p->cache_keep_active > 0 && last_changed[i] >= 0 &&
                                    (step - last_changed[i]) <= p->cache_keep_active;
                if (changed || is_masked[i] || recent) act.push_back(i); else cached.push_back(i);
            }
            if ((int)act.size() >= N || act.empty()) full = true;
        }
        if (full) {
            if (orc_forward_full(md, seq.data(), N, logits_full.data(), use_cache ? &kv : nullptr, n_threads)) return -1;
            if (use_cache) { prev_seq = seq; cache_init = true; }
        } else {
            const int na = (int)act.size();
            std::vector<int32_t> atok(na);
            for (int a = 0; a < na; a++) atok[a] = seq[act[a]];
            std::vector<float> la((size_t)na * V);
            if (orc_forward_cached(md, atok.data(), act.data(), na, N, &kv, cached.data(), la.data(), n_threads)) return -1;
            prev_seq = seq;
            for (int a = 0; a < na; a++)
                memcpy(logits_full.data() + (size_t)act[a] * V, la.data() + (size_t)a * V, (size_t)V * 4);
            rows = na;
        }

        std::vector<orc_candidate> cand;
        for (int i = 0; i < N; i++) {
            if (!is_masked[i]) continue;
            const int lp = shift ? std::max(i - 1, 0) : i;
            const float * row = logits_full.data() + (size_t)lp * V;
            const float ent = orc_entropy(row, V);
            if (p->temperature <= 0.0f) {
                int b; float bv, sv;
                orc_top2(row, V, &b, &bv, &sv);
                const float conf = p->remasking == ORC_REMASK_TOPK_MARGIN ? (bv - sv) : bv;
                cand.push_back({i, b, conf, ent});
            } else {
                float mx = *std::max_element(row, row + V);
                std::vector<float> probs(V);
                float sum = 0.0f;
                for (int v = 0; v < V; v++) { probs[v] = expf((row[v] - mx) / p->temperature); sum += probs[v]; }
                for (int v = 0; v < V; v++) probs[v] /= sum;
                std::discrete_distribution<int> dist(probs.begin(), probs.end());
                const int s = dist(rng);
                cand.push_back({i, s, probs[s], ent});
            }
        }
        int n_unmask = orc_tokens_to_unmask(step, p->n_steps, n_masked, p->schedule);
        if (p->remasking == ORC_REMASK_RANDOM) {
            std::shuffle(cand.begin(), cand.end(), rng);
        } else {
            n_unmask = orc_order_candidates(cand.data(), (int)cand.size(), p->remasking,
                                            p->entropy_threshold, n_unmask);
        }
        int done = 0;
        for (int j = 0; j < n_unmask && j < (int)cand.size(); j++) {
            seq[cand[j].pos] = cand[j].token;
            is_masked[cand[j].pos] = false;
            n_masked--;
            done++;
        }
        if (stats && step < 256) {
            stats->rows_per_step[step] = rows;
            stats->unmasked_per_step[step] = done;
            stats->actual_steps = step + 1;
        }
    }
    memcpy(out, seq.data() + n_prompt, (size_t)n_generate * 4);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Autoregressive path (src/ar-graph.cpp, src/ar-cache.h, src/ar-sampler.cpp)  */
/* ------------------------------------------------------------------------ */
/* Forward of n_new tokens at positions n_past.. over the append-only cache
 * (src/ar-graph.cpp:262-399): keys are cache rows 0..n_past-1 then the new rows,
 * causal mask (+ sliding window), skipped layers leave their cache rows alone.
 * logits: [n_new][V], or only the last row's [V] when last_only. */
extern "C" int orc_ar_forward(const orc_model * md, const int32_t * tokens, int n_new, orc_ar_cache * c,
                              float * logits, int last_only, int profile, int n_threads) {
    if (n_new <= 0 || c->n_past + n_new > c->n_ctx_max) return -1;
    const int d = md->n_embd, L = md->n_layer;
    std::vector<int32_t> pos(n_new), cpos(c->n_past);
    for (int i = 0; i < n_new; i++) pos[i] = c->n_past + i;
    std::iota(cpos.begin(), cpos.end(), 0);
    const orc_kv kv = {c->n_ctx_max, c->k, c->v};
    const size_t per = (size_t)n_new * d;
    std::vector<float> ko(per * L), vo(per * L);
    pass_opts opt;
    opt.causal = true;
    opt.window = c->sliding_window;
    opt.skip = profile ? nullptr : c->skip;
    opt.impact = profile ? c->impact : nullptr;
    opt.head_from = last_only ? n_new - 1 : 0;
    const int rc = run_layers(md, tokens, pos.data(), n_new, c->n_past ? &kv : nullptr, cpos.data(), c->n_past, logits,
                              ko.data(), vo.data(), n_threads, opt);
    if (rc) return rc;
    /* append (src/ar-cache.h:129-155) for the layers that ran */
    const size_t cap = (size_t)c->n_ctx_max * d;
    for (int il = 0; il < L; il++) {
        if (opt.skip && opt.skip[il]) continue;
        memcpy(c->k + il * cap + (size_t)c->n_past * d, ko.data() + il * per, per * 4);
        memcpy(c->v + il * cap + (size_t)c->n_past * d, vo.data() + il * per, per * 4);
    }
    c->n_past += n_new;
    return 0;
}

/* ar_profile_layers' choice (src/ar-graph.cpp:454-505): layers ranked by (impact,
 * index) ascending; the first n_skip outside the two first and two last layers are
 * skipped.  Returns how many were marked. */
extern "C" int orc_ar_choose_skip(const float * impact, int n_layer, int n_skip, uint8_t * skip) {
    memset(skip, 0, (size_t)n_layer);
    if (n_skip <= 0) return 0;
    std::vector<std::pair<float, int>> ranked;
    for (int il = 0; il < n_layer; il++) ranked.push_back({impact[il], il});
    std::sort(ranked.begin(), ranked.end());
    int skipped = 0;
    for (auto & r : ranked) {
        if (skipped >= n_skip) break;
        if (r.second < 2 || r.second >= n_layer - 2) continue;
        skip[r.second] = 1;
        skipped++;
    }
    return skipped;
}

/* sample_token and its filters (src/ar-sampler.cpp:11-140), on a copy of the row. */
static void ar_top_k(float * lg, int V, int top_k) {
    if (top_k <= 0 || top_k >= V) return;
    std::vector<float> tmp(lg, lg + V);
    std::nth_element(tmp.begin(), tmp.begin() + top_k, tmp.end(), std::greater<float>());
    const float threshold = tmp[top_k - 1];
    for (int i = 0; i < V; i++)
        if (lg[i] < threshold) lg[i] = -INFINITY;
}

static void ar_top_p(float * lg, int V, float top_p) {
    if (top_p >= 1.0f) return;
    const float mx = *std::max_element(lg, lg + V);
    float sum = 0.0f;
    for (int i = 0; i < V; i++) { lg[i] = expf(lg[i] - mx); sum += lg[i]; }
    for (int i = 0; i < V; i++) lg[i] /= sum;
    std::vector<int> idx(V);
    std::iota(idx.begin(), idx.end(), 0);
    std::sort(idx.begin(), idx.end(), [&](int a, int b) { return lg[a] > lg[b]; });
    float cum = 0.0f;
    int cutoff = V;
    for (int i = 0; i < V; i++) {
        cum += lg[idx[i]];
        if (cum >= top_p) { cutoff = i + 1; break; }
    }
    for (int i = cutoff; i < V; i++) lg[idx[i]] = 0.0f;
    for (int i = 0; i < V; i++) lg[i] = lg[i] > 0.0f ? logf(lg[i]) : -INFINITY;
}

struct orc_rng { std::mt19937 g; };

extern "C" orc_rng * orc_rng_new(uint32_t seed) { return new orc_rng{std::mt19937(seed)}; }
extern "C" void orc_rng_free(orc_rng * r) { delete r; }

extern "C" int orc_ar_sample(const float * row, int V, const orc_ar_params * p, const int32_t * recent, int n_recent,
                             orc_rng * rng) {
    std::vector<float> lg(row, row + V);
    if (p->repeat_penalty > 1.0f)
        for (int j = 0; j < n_recent; j++) {
            const int32_t t = recent[j];
            if (t >= 0 && t < V) lg[t] = lg[t] > 0.0f ? lg[t] / p->repeat_penalty : lg[t] * p->repeat_penalty;
        }
    if (p->temperature <= 0.0f) {
        int best = 0;
        float bv = lg[0];
        for (int i = 1; i < V; i++)
            if (lg[i] > bv) { bv = lg[i]; best = i; }
        return best;
    }
    for (int i = 0; i < V; i++) lg[i] /= p->temperature;
    ar_top_k(lg.data(), V, p->top_k);
    ar_top_p(lg.data(), V, p->top_p);
    const float mx = *std::max_element(lg.begin(), lg.end());
    float sum = 0.0f;
    std::vector<float> probs(V);
    for (int i = 0; i < V; i++) { probs[i] = expf(lg[i] - mx); sum += probs[i]; }
    for (int i = 0; i < V; i++) probs[i] /= sum;
    std::discrete_distribution<int> dist(probs.begin(), probs.end());
    return dist(rng->g);
}

/* ar_generate (src/ar-sampler.cpp:143-314). */
extern "C" int orc_ar_generate(const orc_model * md, const int32_t * prompt, int n_prompt, int max_tokens,
                               const orc_ar_params * p, int32_t * out, int * n_out, uint8_t * skip_out,
                               int n_threads) {
    const int V = md->n_vocab, L = md->n_layer, d = md->n_embd;
    *n_out = 0;
    /* the reference samples one token from the prefill whatever max_tokens is */
    if (n_prompt <= 0 || max_tokens < 0) return -1;
    orc_ar_cache c;
    c.n_ctx_max = n_prompt + std::max(max_tokens, 1);
    c.n_past = 0;
    c.sliding_window = p->sliding_window;
    std::vector<float> kc((size_t)L * c.n_ctx_max * d, 0.0f), vc((size_t)L * c.n_ctx_max * d, 0.0f);
    std::vector<uint8_t> skip(L, 0);
    std::vector<float> impact(L, 0.0f);
    c.k = kc.data();
    c.v = vc.data();
    c.skip = skip.data();
    c.impact = impact.data();
    std::mt19937 gen(p->seed);
    orc_rng rng{gen};
    std::vector<float> lg(V);
    const bool prof = p->layer_skip > 0;
    if (orc_ar_forward(md, prompt, n_prompt, &c, lg.data(), 1, prof, n_threads)) return -1;
    if (prof) orc_ar_choose_skip(impact.data(), L, p->layer_skip, skip.data());
    if (skip_out) memcpy(skip_out, skip.data(), (size_t)L);
    std::vector<int32_t> recent;
    for (int i = std::max(0, n_prompt - p->repeat_last_n); i < n_prompt; i++) recent.push_back(prompt[i]);
    auto push = [&](int32_t t) {
        out[(*n_out)++] = t;
        recent.push_back(t);
        if ((int)recent.size() > p->repeat_last_n) recent.erase(recent.begin());
    };
    push(orc_ar_sample(lg.data(), V, p, recent.data(), (int)recent.size(), &rng));
    for (int i = 1; i < max_tokens; i++) {
        const int32_t last = out[*n_out - 1];
        if (last == 151643 || last == 151645 || last == 151644) break;   /* src/ar-sampler.cpp:253-260 */
        if (orc_ar_forward(md, &last, 1, &c, lg.data(), 1, 0, n_threads)) return -1;
        push(orc_ar_sample(lg.data(), V, p, recent.data(), (int)recent.size(), &rng));
    }
    return 0;
}
