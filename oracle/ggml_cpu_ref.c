/*
 * ggml_cpu_ref.c -- CPU restatement of ggml-cpu semantics for the quantized
 * decoder path. TEST INFRASTRUCTURE ONLY (the checker); see ggml_cpu_ref.h
 * for the parity status of each function.
 *
 * The block formats, quantizers and dot products follow ggml's published
 * ggml-common.h / ggml-quants.c / ggml-cpu algorithm descriptions (the fork
 * that holds them, openasr-ggml @ 0db3a287, is not vendored in the
 * reference: .gitmodules:1-3). Reference call sites are cited per function.
 */
#include "ggml_cpu_ref.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 -- */

uint16_t ref_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* |f| >= 65520 rounds to infinity */
        return (uint16_t) (sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: half subnormal, unit 2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        const uint32_t m = (uint32_t) rintf(a * 16777216.0f); /* exact scaling, RNE */
        return (uint16_t) (sign | m);
    }
    const uint32_t e = (ax >> 23) - 112u;
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h++;
    }
    return (uint16_t) (sign | h);
}

float ref_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float v = (float) mant * 5.9604644775390625e-8f; /* 2^-24 */
        return sign ? -v : v;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void ref_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ref_fp32_to_fp16(x[i]);
}

void ref_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ref_fp16_to_fp32(x[i]);
}

/* round half to even, as ggml's nearest_int (magic-number add) does */
static inline int nearest_even(float v) { return (int) rintf(v); }

/* ------------------------------------------------- deterministic math -- */

/* exp and sin/cos evaluated in double with a fixed sequence of IEEE
 * operations (no FMA contraction: this file is built with
 * -ffp-contract=off), then rounded once to f32. The device evaluates the
 * identical sequence, so both sides produce the same bits; accuracy is
 * within one rounding of the exact value (checked against libm in the
 * oracle tests). ggml-cpu's own vectorised expf is an ISA-specific
 * approximation of the same function. */
float ref_expf_det(float x) {
    if (x != x) return x;
    if (x > 88.72284f) return INFINITY;
    if (x < -103.97208f) return 0.0f;
    const double xd = (double) x;
    const double k = rint(xd * 1.4426950408889634074);
    const double r = (xd - k * 0.69314718055994528623) - k * 2.3190468138462996154e-17;
    double p = 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return (float) ldexp(p, (int) k);
}

void ref_sincosf_det(float x, float * s_out, float * c_out) {
    const double xd = (double) x;
    const double k = rint(xd * 0.63661977236758134308);
    const double r = (xd - k * 1.5707963267341256458) - k * 6.0771005065061922341e-11;
    const double r2 = r * r;
    double s = -1.0 / 355687428096000.0;
    s = s * r2 + 1.0 / 1307674368000.0;
    s = s * r2 - 1.0 / 6227020800.0;
    s = s * r2 + 1.0 / 39916800.0;
    s = s * r2 - 1.0 / 362880.0;
    s = s * r2 + 1.0 / 5040.0;
    s = s * r2 - 1.0 / 120.0;
    s = s * r2 + 1.0 / 6.0;
    s = r - (r * r2) * s;
    double c = 1.0 / 6402373705728000.0;
    c = c * r2 - 1.0 / 20922789888000.0;
    c = c * r2 + 1.0 / 87178291200.0;
    c = c * r2 - 1.0 / 479001600.0;
    c = c * r2 + 1.0 / 3628800.0;
    c = c * r2 - 1.0 / 40320.0;
    c = c * r2 + 1.0 / 720.0;
    c = c * r2 - 1.0 / 24.0;
    c = c * r2 + 0.5;
    c = 1.0 - r2 * c;
    const int q = (int) (((long long) k) & 3);
    double so, co;
    if (q == 0) { so = s; co = c; }
    else if (q == 1) { so = c; co = -s; }
    else if (q == 2) { so = -s; co = -c; }
    else { so = -c; co = s; }
    *s_out = (float) so;
    *c_out = (float) co;
}

/* ---------------------------------------------------------------- Q8_0 -- */

/* ggml-base quantize_row_q8_0_ref: weights through ggml_quantize_chunk
 * (gguf_write.rs:579-588). d = amax/127, id = 1/d, round half away. */
void ref_quantize_row_q8_0_weights(const float * x, ref_block_q8_0 * y, int64_t k) {
    const int64_t nb = k / REF_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < REF_QK8_0; j++) {
            const float a = fabsf(x[i * REF_QK8_0 + j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = ref_fp32_to_fp16(d);
        for (int j = 0; j < REF_QK8_0; j++) {
            y[i].qs[j] = (int8_t) roundf(x[i * REF_QK8_0 + j] * id);
        }
    }
}

/* ggml-cpu quantize_row_q8_0 on x86 (the activation side of a Q8_0 mul_mat):
 * d = amax/127 stored as f16, multiplier 127/amax, round half to even. */
void ref_quantize_row_q8_0_act(const float * x, ref_block_q8_0 * y, int64_t k) {
    const int64_t nb = k / REF_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < REF_QK8_0; j++) {
            const float a = fabsf(x[i * REF_QK8_0 + j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.0f;
        y[i].d = ref_fp32_to_fp16(d);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < REF_QK8_0; j++) {
            y[i].qs[j] = (int8_t) nearest_even(x[i * REF_QK8_0 + j] * id);
        }
    }
}

void ref_dequantize_row_q8_0(const ref_block_q8_0 * x, float * y, int64_t k) {
    const int64_t nb = k / REF_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float d = ref_fp16_to_fp32(x[i].d);
        for (int j = 0; j < REF_QK8_0; j++) y[i * REF_QK8_0 + j] = x[i].qs[j] * d;
    }
}

/* horizontal sum of eight int32 lanes (integer: order-free) */
static inline int hsum_i32x8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

/* vec_dot_q8_0_q8_0: per block an exact integer dot, scaled by d_x*d_y;
 * block terms summed in f64 and rounded once (see vec_dot_q4_K_q8_K) */
float ref_vec_dot_q8_0_q8_0(int64_t n, const ref_block_q8_0 * x, const ref_block_q8_0 * y) {
    const int64_t nb = n / REF_QK8_0;
    double sum = 0.0;
    for (int64_t i = 0; i < nb; i++) {
        /* the integer dot in AVX2: int8 widened to int16, pair products
         * summed to int32 (exact for every int8 value) */
        const __m256i xv = _mm256_loadu_si256((const __m256i *) x[i].qs);
        const __m256i yv = _mm256_loadu_si256((const __m256i *) y[i].qs);
        const __m256i p0 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm256_castsi256_si128(xv)),
                                             _mm256_cvtepi8_epi16(_mm256_castsi256_si128(yv)));
        const __m256i p1 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm256_extracti128_si256(xv, 1)),
                                             _mm256_cvtepi8_epi16(_mm256_extracti128_si256(yv, 1)));
        const int sumi = hsum_i32x8(_mm256_add_epi32(p0, p1));
        /* d_x*d_y of two halves is exact in f32; the block term is exact in f64 */
        const float dd = ref_fp16_to_fp32(x[i].d) * ref_fp16_to_fp32(y[i].d);
        sum += (double) sumi * (double) dd;
    }
    return (float) sum;
}

/* ---------------------------------------------------------------- Q4_K -- */

/* 6-bit scale/min unpacking of a Q4_K super-block (get_scale_min_k4) */
void ref_get_scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t) ((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void ref_dequantize_row_q4_K(const ref_block_q4_K * x, float * y, int64_t k) {
    const int64_t nb = k / REF_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float d = ref_fp16_to_fp32(x[i].d);
        const float dmin = ref_fp16_to_fp32(x[i].dmin);
        const uint8_t * q = x[i].qs;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            ref_get_scale_min_k4(2 * c, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            ref_get_scale_min_k4(2 * c + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
        }
    }
}

/* ggml's Q4_K weight quantizer, quantize_row_q4_K_ref of ggml-quants.c at
 * the fork's pinned revision (0db3a287511085fb1564fea3f86839f9e40ca39e,
 * model-registry/catalog.public.json:3941), which ggml_quantize_chunk runs
 * for a NULL importance matrix (gguf_write.rs:579-588). The fork is absent
 * from the reference tree; this restates ggml's published algorithm, in
 * float arithmetic in ggml's operation order:
 *  - each 32-weight sub-block is fitted as x ~ scale * L + min (min <= 0,
 *    L in 0..15) by make_qkx2_quants: weights av + |x| (av the sub-block's
 *    RMS); a first fit from the range, then 21 candidate inverse scales
 *    (14 + 0.1 is) / (max - min), each giving L and a weighted least-squares
 *    (scale, min) (min clamped to 0 with the scale refitted), the candidate
 *    of smallest weighted squared error replacing the first fit only when
 *    strictly smaller;
 *  - scales and -mins are coded in 6 bits against the block's largest
 *    (d = max_scale / 63, dmin = max_min / 63 as f16);
 *  - the weights are requantized against the coded values; a sub-block
 *    whose coded scale is 0 keeps the search's L. */
static int q4k_nearest(float v) { return nearest_even(v); }  /* ggml nearest_int: v + 1.5*2^23 */

static float q4k_fit(const float * x, const float * w, uint8_t * L, float * neg_min) {
    enum { n = 32, nmax = 15, nstep = 20 };
    const float rmin = -1.0f, rdelta = 0.1f;
    uint8_t aux[32];
    float lo = x[0], hi = x[0], sw = 0.0f, sx = 0.0f;
    for (int i = 0; i < n; i++) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sw += w[i];
        sx += w[i] * x[i];
    }
    if (lo > 0.0f) lo = 0.0f;
    if (hi == lo) {
        memset(L, 0, n);
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = (float) nmax / (hi - lo);
    float scale = 1.0f / iscale;
    float best = 0.0f;
    for (int i = 0; i < n; i++) {
        int l = q4k_nearest(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t) l;
        const float e = scale * (float) l + lo - x[i];
        best += w[i] * (e * e);
    }
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * (float) is + (float) nmax) / (hi - lo);
        float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;
        for (int i = 0; i < n; i++) {
            int l = q4k_nearest(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            aux[i] = (uint8_t) l;
            const float wl = w[i] * (float) l;
            sl += wl;
            sl2 += wl * (float) l;
            sxl += wl * x[i];
        }
        const float det = sw * sl2 - sl * sl;
        if (!(det > 0.0f)) continue;
        float s = (sw * sxl - sx * sl) / det;
        float m = (sl2 * sx - sl * sxl) / det;
        if (m > 0.0f) {
            m = 0.0f;
            s = sxl / sl2;
        }
        float err = 0.0f;
        for (int i = 0; i < n; i++) {
            const float e = s * (float) aux[i] + m - x[i];
            err += w[i] * (e * e);
        }
        if (err < best) {
            memcpy(L, aux, n);
            best = err;
            scale = s;
            lo = m;
        }
    }
    *neg_min = -lo;
    return scale;
}

void ref_quantize_row_q4_K(const float * x, ref_block_q4_K * y, int64_t k) {
    const int64_t nb = k / REF_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * REF_QK_K;
        uint8_t L[REF_QK_K];
        float scales[8], mins[8], wt[32];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            const float * xs = xb + 32 * j;
            float ss = 0.0f;
            for (int l = 0; l < 32; l++) ss += xs[l] * xs[l];
            const float av = sqrtf(ss / 32.0f);
            for (int l = 0; l < 32; l++) wt[l] = av + fabsf(xs[l]);
            scales[j] = q4k_fit(xs, wt, L + 32 * j, &mins[j]);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            const int a = q4k_nearest(inv_scale * scales[j]);
            const int b = q4k_nearest(inv_min * mins[j]);
            ls[j] = (uint8_t) (a > 63 ? 63 : a);
            lm[j] = (uint8_t) (b > 63 ? 63 : b);
        }
        memset(y[i].scales, 0, 12);
        for (int j = 0; j < 4; j++) {
            y[i].scales[j] = (uint8_t) (ls[j] | ((ls[j + 4] >> 4) << 6));
            y[i].scales[j + 4] = (uint8_t) (lm[j] | ((lm[j + 4] >> 4) << 6));
            y[i].scales[j + 8] = (uint8_t) ((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
        }
        y[i].d = ref_fp32_to_fp16(max_scale / 63.0f);
        y[i].dmin = ref_fp32_to_fp16(max_min / 63.0f);
        const float d = ref_fp16_to_fp32(y[i].d);
        const float dmin = ref_fp16_to_fp32(y[i].dmin);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            ref_get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float dd = d * (float) sc;
            if (dd == 0.0f) continue;  /* keeps the search's L */
            const float dm = dmin * (float) m;
            for (int l = 0; l < 32; l++) {
                int q = q4k_nearest((xb[32 * j + l] + dm) / dd);
                L[32 * j + l] = (uint8_t) (q < 0 ? 0 : (q > 15 ? 15 : q));
            }
        }
        for (int c = 0; c < 4; c++) {
            for (int l = 0; l < 32; l++) {
                y[i].qs[32 * c + l] = (uint8_t) (L[64 * c + l] | (L[64 * c + 32 + l] << 4));
            }
        }
    }
}

/* ---------------------------------------------------------------- Q8_K -- */

/* quantize_row_q8_K_ref: iscale = -127/max where max is the signed value of
 * largest magnitude; d = 1/iscale; bsums over groups of 16. */
void ref_quantize_row_q8_K(const float * x, ref_block_q8_K * y, int64_t k) {
    const int64_t nb = k / REF_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * REF_QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < REF_QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (amax == 0.0f) {
            y[i].d = 0.0f;
            memset(y[i].qs, 0, REF_QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < REF_QK_K; j++) {
            const int v = nearest_even(iscale * xb[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < REF_QK_K / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t) s;
        }
        y[i].d = 1.0f / iscale;
    }
}

void ref_dequantize_row_q8_K(const ref_block_q8_K * x, float * y, int64_t k) {
    const int64_t nb = k / REF_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        for (int j = 0; j < REF_QK_K; j++) y[i * REF_QK_K + j] = x[i].d * x[i].qs[j];
    }
}

/* vec_dot_q4_K_q8_K: per super-block the scaled integer sum and the mins
 * correction (through the Q8_K bsums) are exact integers; the super-block
 * term d*isum - dmin*msum is formed in f64 and the terms are summed in f64,
 * rounding to f32 once. ggml-cpu sums the same terms in f32 SIMD lanes (an
 * ISA-dependent order); summing wide makes the result independent of order,
 * so any correct device reduction reproduces it bit for bit. */
float ref_vec_dot_q4_K_q8_K(int64_t n, const ref_block_q4_K * x, const ref_block_q8_K * y) {
    const int64_t nb = n / REF_QK_K;
    double sum = 0.0;
    for (int64_t i = 0; i < nb; i++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) ref_get_scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        int msum = 0;
        for (int j = 0; j < 16; j++) msum += (int) y[i].bsums[j] * (int) mn[j / 2];
        /* isum = sum_c sc[2c] * <lo nibbles, q8[64c..+32]> + sc[2c+1] * <hi
         * nibbles, q8[64c+32..+32]>, in AVX2: unsigned nibble x int8 pairs
         * (|pair| <= 2*15*128, no int16 saturation), then x the 6-bit scale
         * into int32 lanes; exact integer arithmetic */
        const uint8_t * q4 = x[i].qs;
        const int8_t * q8 = y[i].qs;
        const __m256i m4 = _mm256_set1_epi8(0x0F);
        __m256i acc = _mm256_setzero_si256();
        for (int c = 0; c < 4; c++) {
            const __m256i q4v = _mm256_loadu_si256((const __m256i *) (q4 + 32 * c));
            const __m256i lo = _mm256_and_si256(q4v, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q4v, 4), m4);
            const __m256i y0 = _mm256_loadu_si256((const __m256i *) (q8 + 64 * c));
            const __m256i y1 = _mm256_loadu_si256((const __m256i *) (q8 + 64 * c + 32));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_maddubs_epi16(lo, y0), _mm256_set1_epi16(sc[2 * c])));
            acc = _mm256_add_epi32(acc,
                                   _mm256_madd_epi16(_mm256_maddubs_epi16(hi, y1), _mm256_set1_epi16(sc[2 * c + 1])));
        }
        const int isum = hsum_i32x8(acc);
        const double d = (double) ref_fp16_to_fp32(x[i].d) * (double) y[i].d;
        const double dmin = (double) ref_fp16_to_fp32(x[i].dmin) * (double) y[i].d;
        sum += d * (double) isum - dmin * (double) msum;
    }
    return (float) sum;
}

/* ---------------------------------------------------------------- Q3_K -- */
/* The Q3_K weight format, written by the host's pack writer for decoder
 * matrices under the q3_k pack policy (models/pack_quant.rs:205-207, through
 * ggml_quantize_chunk, ggml_runtime/gguf_write.rs:579-588) and multiplied by
 * ggml-cpu's MUL_MAT against Q8_K activations. ggml-base's published layout
 * (block_q3_K, dequantize_row_q3_K, vec_dot_q3_K_q8_K of the fork's pinned
 * revision 0db3a287): weight e = 128h + 32j + l of a super-block (h < 2,
 * j < 4, l < 32) is d * (scale[8h + 2j + l/16] - 32) * q with
 * q = ((qs[32h + l] >> 2j) & 3) - (hmask[l] bit 4h + j ? 0 : 4). */

/* 6-bit scale i of 16: the low four bits are nibble i/8 of byte i%8, the
 * high two bits are bits 2(i/4)..+1 of byte 8 + i%4 */
int ref_q3_K_scale(const uint8_t * scales, int i) {
    const int lo = (scales[i % 8] >> (4 * (i / 8))) & 0xF;
    const int hi = (scales[8 + i % 4] >> (2 * (i / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}

static inline int q3_K_quant(const ref_block_q3_K * b, int e) {
    const int h = e / 128, j = (e % 128) / 32, l = e % 32;
    const int q = (b->qs[32 * h + l] >> (2 * j)) & 3;
    return q - ((b->hmask[l] >> (4 * h + j)) & 1 ? 0 : 4);
}

void ref_dequantize_row_q3_K(const ref_block_q3_K * x, float * y, int64_t k) {
    const int64_t nb = k / REF_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float d = ref_fp16_to_fp32(x[i].d);
        for (int e = 0; e < REF_QK_K; e++) {
            const float dl = d * (float) ref_q3_K_scale(x[i].scales, e / 16);
            y[i * REF_QK_K + e] = dl * (float) q3_K_quant(&x[i], e);
        }
    }
}

/* vec_dot_q3_K_q8_K: per super-block isum = sum over the sixteen 16-weight
 * groups of (scale - 32) * <q, q8>, an exact integer; the term
 * d_x * d_y * isum is exact in f64 and the terms are summed in f64, rounding
 * to f32 once (ggml-cpu sums them in ISA-dependent f32 lanes; the wide sum
 * makes the value independent of the order, as for Q4_K) */
float ref_vec_dot_q3_K_q8_K(int64_t n, const ref_block_q3_K * x, const ref_block_q8_K * y) {
    const int64_t nb = n / REF_QK_K;
    double sum = 0.0;
    for (int64_t i = 0; i < nb; i++) {
        int64_t isum = 0;
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += q3_K_quant(&x[i], 16 * g + l) * (int) y[i].qs[16 * g + l];
            isum += (int64_t) ref_q3_K_scale(x[i].scales, g) * s;
        }
        sum += (double) ref_fp16_to_fp32(x[i].d) * (double) y[i].d * (double) isum;
    }
    return (float) sum;
}

/* ggml_vec_dot_f16: products of two halves are exact in f32; summed wide */
float ref_vec_dot_f16(int64_t n, const uint16_t * x, const uint16_t * y) {
    double s = 0.0;
    for (int64_t i = 0; i < n; i++) s += (double) (ref_fp16_to_fp32(x[i]) * ref_fp16_to_fp32(y[i]));
    return (float) s;
}

size_t ref_row_size(int type, int64_t ne0) {
    switch (type) {
        case REF_F32: return (size_t) ne0 * 4;
        case REF_F16: return (size_t) ne0 * 2;
        case REF_Q8_0: return (size_t) (ne0 / REF_QK8_0) * sizeof(ref_block_q8_0);
        case REF_Q4_K: return (size_t) (ne0 / REF_QK_K) * sizeof(ref_block_q4_K);
        case REF_Q3_K: return (size_t) (ne0 / REF_QK_K) * sizeof(ref_block_q3_K);
        case REF_Q8_K: return (size_t) (ne0 / REF_QK_K) * sizeof(ref_block_q8_K);
        default: return 0;
    }
}

/* ------------------------------------------------------------- mul_mat -- */

void ref_mul_mat(int wtype, const void * w, size_t row_bytes, int64_t m, int64_t k,
                 const float * x, int64_t x_stride, int64_t n, float * dst, int64_t d_stride,
                 int n_threads) {
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
#else
    (void) n_threads;
#endif
    /* every column is converted to the weight's vec_dot type once, then each
     * weight row is streamed once against all columns (ggml-cpu's "convert
     * src1 first" rule; the loop order only changes speed, not results) */
    const int vtype = wtype == REF_Q8_0 ? REF_Q8_0
                      : (wtype == REF_Q4_K || wtype == REF_Q3_K) ? REF_Q8_K
                      : (wtype == REF_F16 ? REF_F16 : REF_F32);
    const size_t qrow = vtype == REF_F32 ? (size_t) k * 4 : ref_row_size(vtype, k);
    char * xq = (char *) malloc(qrow * (size_t) (n > 0 ? n : 1));
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t col = 0; col < n; col++) {
        const float * xc = x + col * x_stride;
        char * o = xq + (size_t) col * qrow;
        if (vtype == REF_Q8_0) ref_quantize_row_q8_0_act(xc, (ref_block_q8_0 *) o, k);
        else if (vtype == REF_Q8_K) ref_quantize_row_q8_K(xc, (ref_block_q8_K *) o, k);
        else if (vtype == REF_F16) ref_fp32_to_fp16_row(xc, (uint16_t *) o, k);
        else memcpy(o, xc, (size_t) k * 4);
    }
#pragma omp parallel for num_threads(n_threads) schedule(dynamic, 16)
    for (int64_t r = 0; r < m; r++) {
        const char * wr = (const char *) w + r * row_bytes;
        for (int64_t col = 0; col < n; col++) {
            const char * xc = xq + (size_t) col * qrow;
            float v;
            if (vtype == REF_Q8_0) {
                v = ref_vec_dot_q8_0_q8_0(k, (const ref_block_q8_0 *) wr, (const ref_block_q8_0 *) xc);
            } else if (wtype == REF_Q3_K) {
                v = ref_vec_dot_q3_K_q8_K(k, (const ref_block_q3_K *) wr, (const ref_block_q8_K *) xc);
            } else if (vtype == REF_Q8_K) {
                v = ref_vec_dot_q4_K_q8_K(k, (const ref_block_q4_K *) wr, (const ref_block_q8_K *) xc);
            } else if (vtype == REF_F16) {
                v = ref_vec_dot_f16(k, (const uint16_t *) wr, (const uint16_t *) xc);
            } else { /* ggml_vec_dot_f32 */
                const float * a = (const float *) wr;
                const float * b = (const float *) xc;
                double s = 0.0;
                for (int64_t i = 0; i < k; i++) s += (double) (a[i] * b[i]);
                v = (float) s;
            }
            dst[col * d_stride + r] = v;
        }
    }
    free(xq);
}

/* ---------------------------------------------------------- row ops ---- */

/* ggml_compute_forward_rms_norm_f32 (nn/norm.rs:39-56): double sum of x*x */
void ref_rms_norm(const float * x, float * y, int64_t ne0, int64_t rows, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        const float * xr = x + r * ne0;
        float * yr = y + r * ne0;
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; i++) sum += (double) (xr[i] * xr[i]);
        const float mean = (float) (sum / ne0);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < ne0; i++) yr[i] = xr[i] * scale;
    }
}

/* ggml_compute_forward_norm_f32 (nn/norm.rs:10-33): mean, then variance */
void ref_norm(const float * x, float * y, int64_t ne0, int64_t rows, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        const float * xr = x + r * ne0;
        float * yr = y + r * ne0;
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; i++) sum += (double) xr[i];
        const float mean = (float) (sum / ne0);
        double sum2 = 0.0;
        for (int64_t i = 0; i < ne0; i++) {
            const float v = xr[i] - mean;
            yr[i] = v;
            sum2 += (double) (v * v);
        }
        const float variance = (float) (sum2 / ne0);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < ne0; i++) yr[i] *= scale;
    }
}

float ref_silu(float x) { return x / (1.0f + ref_expf_det(-x)); }

/* erf as a fixed sequence of double operations rounded once: the Maclaurin
 * series 2/sqrt(pi) x sum_{n < 64} a_n (x^2)^n with a_n = (-1)^n / (n!
 * (2n+1)) rounded to the nearest double, evaluated by Horner's rule from n =
 * 63 down (separate multiply and add), for |x| < 4; +-1 beyond (where erf
 * rounds to +-1 in f32). ggml-cpu's GELU_ERF (ggml_vec_gelu_erf_f32) calls
 * libm erff, which is not reproducible across devices; this sequence is, and
 * it is pinned against math.erf. The device runs the same table and steps. */
static const double kErfCoef[64] = {
    0x1.0000000000000p+0, -0x1.5555555555555p-2, 0x1.999999999999ap-4, -0x1.8618618618618p-6,
    0x1.2f684bda12f68p-8, -0x1.8d3018d3018d3p-11, 0x1.c01c01c01c01cp-14, -0x1.bbd779334ef0bp-17,
    0x1.87a00187a0018p-20, -0x1.3777c55568ccdp-23, 0x1.c2e3054870b38p-27, -0x1.2b67310aa9f3ap-30,
    0x1.6f448e13e85e1p-34, -0x1.a289ee7e40f74p-38, 0x1.bd577e658d020p-42, -0x1.bc6250fb14231p-46,
    0x1.a173a167fba4dp-50, -0x1.7271cbe5863ecp-54, 0x1.377c2110f2083p-58, -0x1.f1b4073b34a68p-63,
    0x1.7abd72258fb6ep-67, -0x1.13246abce1bddp-71, 0x1.7e6b81382cd42p-76, -0x1.fd6bebd65107ap-81,
    0x1.45c0a838efe59p-85, -0x1.909c9de3a31c5p-90, 0x1.da7460554e5dbp-95, -0x1.0eef30fa10d2cp-99,
    0x1.2ac65385f79acp-104, -0x1.3e81bb5701ac5p-109, 0x1.4899fcdef0a8dp-114, -0x1.486eea20c2656p-119,
    0x1.3e53defc4e233p-124, -0x1.2b778acc3dedfp-129, 0x1.11ae81077a49ep-134, -0x1.e6597092ccbf0p-140,
    0x1.a47767f2a3c32p-145, -0x1.61f30bc3acd1ap-150, 0x1.22521d98f98a9p-155, -0x1.d05cc9e3507c9p-161,
    0x1.6a513f56f8a2fp-166, -0x1.13f85fc9e143ep-171, 0x1.9aa19d4d16643p-177, -0x1.2a8fa59ffec31p-182,
    0x1.a8830736a5123p-188, -0x1.273d8edcec957p-193, 0x1.91ef82b367a95p-199, -0x1.0be5a4cd94283p-204,
    0x1.5dd4c9219115ap-210, -0x1.bfb10e0f68c50p-216, 0x1.18d952ef00889p-221, -0x1.59982b2e94840p-227,
    0x1.a13ec00b39f6fp-233, -0x1.ee6cefaa5a158p-239, 0x1.1f9dec94da5f8p-244, -0x1.48a6b3820b441p-250,
    0x1.70f41ac13e2a1p-256, -0x1.970f1cb2ad53fp-262, 0x1.b97d90d3e603bp-268, -0x1.d6db2a7c68dcbp-274,
    0x1.edf1e6e4658a9p-280, -0x1.fdcf88bbf71dbp-286, 0x1.02eb04e5f82f5p-291, -0x1.02e2bc1b5790ep-297,
};

double ref_erf_coef(int n) { return kErfCoef[n]; }

float ref_erff_det(float x) {
    if (x != x) return x;
    const double xd = (double) x;
    if (xd >= 4.0) return 1.0f;
    if (xd <= -4.0) return -1.0f;
    const double t = xd * xd;
    double p = kErfCoef[63];
    for (int n = 62; n >= 0; n--) p = p * t + kErfCoef[n];
    return (float) (xd * p * 1.1283791670955125739);
}

/* ggml_vec_gelu_erf_f32: 0.5 x (1 + erf(x / sqrt 2)) in f32 */
float ref_gelu_erf(float x) { return 0.5f * x * (1.0f + ref_erff_det(x * 0.70710678118654752440f)); }

float ref_relu(float x) { return x > 0.0f ? x : 0.0f; }

float ref_gelu_f32(float x) {
    const float c = 0.79788456080286535587989211986876f; /* sqrt(2/pi) */
    return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + 0.044715f * x * x)));
}

/* ggml-cpu GELU goes through a table indexed by the f16 bits of x, holding
 * f16(gelu(f16 x)); |x| >= 10 short-circuits (ggml_vec_gelu_f32). */
float ref_gelu(float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    const float xh = ref_fp16_to_fp32(ref_fp32_to_fp16(x));
    return ref_fp16_to_fp32(ref_fp32_to_fp16(ref_gelu_f32(xh)));
}

/* ggml_compute_forward_rope_f32, NEOX mode, ext_factor 0, attn_factor 1
 * (cpu_graph.rs:1135-1161): theta advances by repeated multiplication with
 * theta_scale = freq_base^(-2/n_dims), as ggml_rope_cache_init does. */
void ref_rope_neox(const float * x, float * y, int64_t head_dim, int64_t n_heads, int64_t n_tokens,
                   const int32_t * pos, int n_dims, float freq_base, float freq_scale) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    float * cache = (float *) malloc(sizeof(float) * (size_t) n_dims);
    for (int64_t t = 0; t < n_tokens; t++) {
        float theta = (float) pos[t];
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const float th = freq_scale * theta;
            ref_sincosf_det(th, &cache[i0 + 1], &cache[i0]);
            theta *= theta_scale;
        }
        for (int64_t h = 0; h < n_heads; h++) {
            const float * xr = x + (t * n_heads + h) * head_dim;
            float * yr = y + (t * n_heads + h) * head_dim;
            const int half = n_dims / 2;
            for (int ic = 0; ic < half; ic++) {
                const float c = cache[2 * ic], s = cache[2 * ic + 1];
                const float x0 = xr[ic], x1 = xr[ic + half];
                yr[ic] = x0 * c - x1 * s;
                yr[ic + half] = x0 * s + x1 * c;
            }
            for (int64_t i = n_dims; i < head_dim; i++) yr[i] = xr[i];
        }
    }
    free(cache);
}

/* ggml_compute_forward_soft_max_f32 with an f16 mask, max_bias 0 */
void ref_soft_max_ext(const float * x, const uint16_t * mask, float * y, int64_t ne0, int64_t rows,
                      float scale) {
    float * wp = (float *) malloc(sizeof(float) * (size_t) ne0);
    for (int64_t r = 0; r < rows; r++) {
        float mx = -INFINITY;
        for (int64_t i = 0; i < ne0; i++) {
            wp[i] = x[r * ne0 + i] * scale + (mask ? ref_fp16_to_fp32(mask[r * ne0 + i]) : 0.0f);
            mx = wp[i] > mx ? wp[i] : mx;
        }
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; i++) {
            const float e = ref_expf_det(wp[i] - mx);
            y[r * ne0 + i] = e;
            sum += (double) e;
        }
        const float inv = (float) (1.0 / sum);
        for (int64_t i = 0; i < ne0; i++) y[r * ne0 + i] *= inv;
    }
    free(wp);
}

/* ggml_vec_argmax_f32 keeps the LAST index equal to the running max; the
 * host relies on this when it reverses logits (cpu_graph.rs:3770-3772). */
int32_t ref_argmax_last(const float * x, int64_t n) {
    float mx = -INFINITY;
    int32_t idx = 0;
    for (int64_t i = 0; i < n; i++) {
        mx = x[i] > mx ? x[i] : mx;
        idx = x[i] == mx ? (int32_t) i : idx;
    }
    return idx;
}

/* first-max rule of OpenASR greedy selection (device_greedy_token.rs:44-75,
 * whisper/ggml_decoder_graph.rs:6232-6240) */
int32_t ref_argmax_first(const float * x, int64_t n) {
    float mx = -INFINITY;
    int32_t idx = 0;
    for (int64_t i = 0; i < n; i++) {
        if (x[i] > mx) {
            mx = x[i];
            idx = (int32_t) i;
        }
    }
    return idx;
}

/* ----------------------------------------------------- flash attention -- */

/* s[j] = sum_d (double) (k_j[d] * q[d]) for up to four positions j, each
 * summed in dim order (the f32 products are exact roundings of the f16
 * operands' products; F16C converts f16 exactly). Four positions are in
 * flight so the dependent f64 adds of one sum overlap the others'. */
static void fa_dot4(const uint16_t * k, int64_t kv_stride_pos, const float * qf, int64_t D, int n, double * s) {
    float tt[512][4];
    for (int j = 0; j < 4; j++) {
        if (j >= n) {
            for (int64_t d = 0; d < D; d++) tt[d][j] = 0.0f;
            continue;
        }
        const uint16_t * kr = k + j * kv_stride_pos;
        for (int64_t d = 0; d < D; d += 8) {
            float pr[8];
            _mm256_storeu_ps(pr, _mm256_mul_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (kr + d))),
                                               _mm256_loadu_ps(qf + d)));
            for (int e = 0; e < 8; e++) tt[d + e][j] = pr[e];
        }
    }
    __m256d a = _mm256_setzero_pd();
    for (int64_t d = 0; d < D; d++) a = _mm256_add_pd(a, _mm256_cvtps_pd(_mm_loadu_ps(tt[d])));
    _mm256_storeu_pd(s, a);
}

/* fidelity 4 for one (query, head): fixed 64-position KV chunks, each with
 * its own max m_c, p = exp(s - m_c), f64 sums l_c and a_c; the chunks are
 * combined in order with w = exp(m_c - M), M = max m_c. Masked (-inf)
 * positions contribute nothing. Scores are formed once and kept. */
static void fa_chunked_one(const uint16_t * qh, const uint16_t * k, const uint16_t * v, int64_t kv_stride_pos,
                           const uint16_t * mask, float * o, int64_t D, int64_t n_kv, float scale) {
    const int64_t C = 64, n_chunks = (n_kv + C - 1) / C;
    if (n_chunks > 1024) abort(); /* spans beyond 65536 positions are not modelled */
    if (D % 8 != 0 || D > 512) abort();
    float qf[512];
    for (int64_t d = 0; d < D; d++) qf[d] = ref_fp16_to_fp32(qh[d]);
    float * sc = (float *) malloc((size_t) (n_kv > 0 ? n_kv : 1) * sizeof(float));
    float mcs[1024];
    float M = -INFINITY;
    for (int64_t c = 0; c < n_chunks; c++) {
        float mc = -INFINITY;
        const int64_t e = n_kv < (c + 1) * C ? n_kv : (c + 1) * C;
        for (int64_t i0 = c * C; i0 < e; i0 += 4) {
            const int n = e - i0 < 4 ? (int) (e - i0) : 4;
            float mv[4];
            int live = 0;
            for (int j = 0; j < n; j++) {
                mv[j] = mask ? ref_fp16_to_fp32(mask[i0 + j]) : 0.0f;
                live |= mv[j] != -INFINITY;
            }
            double a[4] = {0.0, 0.0, 0.0, 0.0};
            if (live) fa_dot4(k + i0 * kv_stride_pos, kv_stride_pos, qf, D, n, a);
            for (int j = 0; j < n; j++) {
                if (mv[j] == -INFINITY) {
                    sc[i0 + j] = -INFINITY;
                    continue;
                }
                const float s = (float) a[j] * scale + mv[j];
                sc[i0 + j] = s;
                mc = s > mc ? s : mc;
            }
        }
        mcs[c] = mc;
        M = mc > M ? mc : M;
    }
    double L = 0.0;
    double O[512], acc[512];
    for (int64_t d = 0; d < D; d++) O[d] = 0.0;
    for (int64_t c = 0; c < n_chunks && M != -INFINITY; c++) {
        if (mcs[c] == -INFINITY) continue;
        const float w = ref_expf_det(mcs[c] - M);
        if (w == 0.0f) continue;
        double l = 0.0;
        for (int64_t d = 0; d < D; d++) acc[d] = 0.0;
        const int64_t e = n_kv < (c + 1) * C ? n_kv : (c + 1) * C;
        for (int64_t ic = c * C; ic < e; ic++) {
            if (sc[ic] == -INFINITY) continue;
            const float p = ref_expf_det(sc[ic] - mcs[c]);
            l += (double) p;
            if (p == 0.0f) continue;
            /* acc[d] += p * v[d], per d in position order (f32 x f32 exact in f64) */
            const uint16_t * vr = v + ic * kv_stride_pos;
            const __m256d p4 = _mm256_set1_pd((double) p);
            for (int64_t d = 0; d < D; d += 8) {
                const __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (vr + d)));
                const __m256d lo = _mm256_mul_pd(p4, _mm256_cvtps_pd(_mm256_castps256_ps128(vf)));
                const __m256d hi = _mm256_mul_pd(p4, _mm256_cvtps_pd(_mm256_extractf128_ps(vf, 1)));
                _mm256_storeu_pd(acc + d, _mm256_add_pd(_mm256_loadu_pd(acc + d), lo));
                _mm256_storeu_pd(acc + d + 4, _mm256_add_pd(_mm256_loadu_pd(acc + d + 4), hi));
            }
        }
        L += (double) w * l;
        for (int64_t d = 0; d < D; d++) O[d] += (double) w * acc[d];
    }
    for (int64_t d = 0; d < D; d++) o[d] = L == 0.0 ? 0.0f : (float) (O[d] / L);
    free(sc);
}

/* s[j] for up to eight positions j: one f32 fused multiply-add chain per
 * position over the dims in order, acc = fma(k_j[d], q[d], acc) from 0 (F16C
 * converts f16 exactly; each vector lane carries one position's chain, so
 * the vector form gives the scalar chain's bits). */
static void fa5_dot8(const uint16_t * k, int64_t kv_stride_pos, const float * qf, int64_t D, int n, float * s) {
    float tt[512][8];
    for (int j = 0; j < 8; j++) {
        if (j >= n) {
            for (int64_t d = 0; d < D; d++) tt[d][j] = 0.0f;
            continue;
        }
        const uint16_t * kr = k + j * kv_stride_pos;
        for (int64_t d = 0; d < D; d += 8) {
            float pr[8];
            _mm256_storeu_ps(pr, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (kr + d))));
            for (int e = 0; e < 8; e++) tt[d + e][j] = pr[e];
        }
    }
    __m256 a = _mm256_setzero_ps();
    for (int64_t d = 0; d < D; d++) a = _mm256_fmadd_ps(_mm256_loadu_ps(tt[d]), _mm256_set1_ps(qf[d]), a);
    _mm256_storeu_ps(s, a);
}

/* fidelity 5 for one (query, head): fixed 64-position KV chunks; per live
 * (unmasked) position the score is the f32 fma chain over dims times scale
 * plus the mask value; per chunk m_c = max s, p = exp(s - m_c), and in
 * position order l_c = l_c + p and a_c[d] = fma(p, v[d], a_c[d]) in f32
 * (every live position, p = 0 included); masked positions are skipped. The
 * chunks are combined in order in f64 with w = exp(m_c - M), M = max m_c:
 * L += w * l_c, O += w * a_c, out = O / L rounded once. */
static void fa_chunked5_one(const uint16_t * qh, const uint16_t * k, const uint16_t * v, int64_t kv_stride_pos,
                            const uint16_t * mask, float * o, int64_t D, int64_t n_kv, float scale) {
    const int64_t C = 64, n_chunks = (n_kv + C - 1) / C;
    if (n_chunks > 1024) abort(); /* spans beyond 65536 positions are not modelled */
    if (D % 8 != 0 || D > 512) abort();
    float qf[512];
    for (int64_t d = 0; d < D; d++) qf[d] = ref_fp16_to_fp32(qh[d]);
    float * sc = (float *) malloc((size_t) (n_kv > 0 ? n_kv : 1) * sizeof(float));
    float mcs[1024];
    float M = -INFINITY;
    for (int64_t c = 0; c < n_chunks; c++) {
        float mc = -INFINITY;
        const int64_t e = n_kv < (c + 1) * C ? n_kv : (c + 1) * C;
        for (int64_t i0 = c * C; i0 < e; i0 += 8) {
            const int n = e - i0 < 8 ? (int) (e - i0) : 8;
            float mv[8];
            int live = 0;
            for (int j = 0; j < n; j++) {
                mv[j] = mask ? ref_fp16_to_fp32(mask[i0 + j]) : 0.0f;
                live |= mv[j] != -INFINITY;
            }
            float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            if (live) fa5_dot8(k + i0 * kv_stride_pos, kv_stride_pos, qf, D, n, a);
            for (int j = 0; j < n; j++) {
                if (mv[j] == -INFINITY) {
                    sc[i0 + j] = -INFINITY;
                    continue;
                }
                const float s = a[j] * scale + mv[j];
                sc[i0 + j] = s;
                mc = s > mc ? s : mc;
            }
        }
        mcs[c] = mc;
        M = mc > M ? mc : M;
    }
    double L = 0.0;
    double O[512];
    float acc[512];
    for (int64_t d = 0; d < D; d++) O[d] = 0.0;
    for (int64_t c = 0; c < n_chunks && M != -INFINITY; c++) {
        if (mcs[c] == -INFINITY) continue;
        const float w = ref_expf_det(mcs[c] - M);
        if (w == 0.0f) continue;
        float l = 0.0f;
        for (int64_t d = 0; d < D; d++) acc[d] = 0.0f;
        const int64_t e = n_kv < (c + 1) * C ? n_kv : (c + 1) * C;
        for (int64_t ic = c * C; ic < e; ic++) {
            if (sc[ic] == -INFINITY) continue;
            const float p = ref_expf_det(sc[ic] - mcs[c]);
            l = l + p;
            const uint16_t * vr = v + ic * kv_stride_pos;
            const __m256 p8 = _mm256_set1_ps(p);
            for (int64_t d = 0; d < D; d += 8) {
                const __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (vr + d)));
                _mm256_storeu_ps(acc + d, _mm256_fmadd_ps(p8, vf, _mm256_loadu_ps(acc + d)));
            }
        }
        L += (double) w * (double) l;
        for (int64_t d = 0; d < D; d++) O[d] += (double) w * (double) acc[d];
    }
    for (int64_t d = 0; d < D; d++) o[d] = L == 0.0 ? 0.0f : (float) (O[d] / L);
    free(sc);
}

/* The unfused attention chain of llm_naive_masked_attention
 * (crates/openasr-core/src/nn/decoder.rs:2154-2200), the attention the host
 * emits on a discrete GPU for prefill chunks of more than two queries over a
 * span of more than 32 positions (models/qwen/llm_transformer.rs:7864-7877):
 *   S = MUL_MAT(K, Q)                  per (position t, query, head)
 *   P = SOFT_MAX_EXT(S, mask, scale)   over the positions of a row
 *   O = MUL_MAT(CONT(TRANSPOSE(V)), P), PERMUTE(0, 2, 1, 3), CONT
 * GQA is MUL_MAT's batch broadcast: query head h reads kv head h / (Hq/Hkv),
 * which is also what the REPEAT-expanded K/V of expand_attention_kv
 * (nn/decoder.rs:1799-1841) hold. prec_f32: the GGML_PREC_F32 the host sets
 * on both products for an F16 src0 with an F32 src1 on CUDA/HIP backends
 * (ggml_runtime/cpu_graph.rs:157-165, 202-228, 3638-3686): Q and P stay f32;
 * without it they are rounded to f16, as ggml-cpu converts src1 to an F16
 * src0's vec_dot type. The arithmetic is defined as:
 *   score: one f32 fused multiply-add chain over the dims in order,
 *          acc = fma(k[d], q[d], acc) from +0; then s = acc * scale + mask
 *          (two roundings, soft_max's scale then mask add); a masked (-inf)
 *          position is -inf without its dot;
 *   softmax: M = max s; e = exp(s - M) (the deterministic exp); the f64 sum
 *          of e over each 64-position chunk by a pairwise tree (level k adds
 *          neighbouring sums of 2^k positions, positions past the span add
 *          +0), then of the chunk sums in chunk order from 0;
 *          P = e * (float) (1 / sum);
 *   context: out[d] = fma(P[t], v[t][d], out[d]) over t in order from +0
 *          (terms with P = 0 are skipped: they leave a sum that is never -0
 *          unchanged).
 * out: [n_q][Hq][D], the CONT of the permuted context. */
void ref_naive_attention(const float * q, int64_t q_stride_tok, int64_t q_stride_head, const uint16_t * k,
                         const uint16_t * v, int64_t kv_stride_head, int64_t kv_stride_pos, const uint16_t * mask,
                         int64_t mask_stride, float * out, int64_t D, int64_t n_q, int64_t Hq, int64_t Hkv,
                         int64_t n_kv, float scale, int prec_f32, int n_threads) {
    const int64_t group = Hq / Hkv, C = 64;
    if (D % 8 != 0 || D > 512) abort();
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
#else
    (void) n_threads;
#endif
#pragma omp parallel for collapse(2) num_threads(n_threads) schedule(static)
    for (int64_t iq = 0; iq < n_q; iq++) {
        for (int64_t h = 0; h < Hq; h++) {
            const int64_t kvh = h / group;
            const uint16_t * kb = k + kvh * kv_stride_head;
            const uint16_t * vb = v + kvh * kv_stride_head;
            const uint16_t * mr = mask ? mask + iq * mask_stride : NULL;
            const float * qr = q + iq * q_stride_tok + h * q_stride_head;
            float qf[512];
            for (int64_t d = 0; d < D; d++) qf[d] = prec_f32 ? qr[d] : ref_fp16_to_fp32(ref_fp32_to_fp16(qr[d]));
            float * sc = (float *) malloc((size_t) (n_kv > 0 ? n_kv : 1) * sizeof(float));
            float M = -INFINITY;
            for (int64_t i0 = 0; i0 < n_kv; i0 += 8) {
                const int n = n_kv - i0 < 8 ? (int) (n_kv - i0) : 8;
                float mv[8];
                int live = 0;
                for (int j = 0; j < n; j++) {
                    mv[j] = mr ? ref_fp16_to_fp32(mr[i0 + j]) : 0.0f;
                    live |= mv[j] != -INFINITY;
                }
                float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                if (live) fa5_dot8(kb + i0 * kv_stride_pos, kv_stride_pos, qf, D, n, a);
                for (int j = 0; j < n; j++) {
                    sc[i0 + j] = mv[j] == -INFINITY ? -INFINITY : a[j] * scale + mv[j];
                    M = sc[i0 + j] > M ? sc[i0 + j] : M;
                }
            }
            double sum = 0.0;
            for (int64_t c0 = 0; c0 < n_kv; c0 += C) {
                double tree[64];
                for (int64_t j = 0; j < C; j++) {
                    const int64_t t = c0 + j;
                    if (t < n_kv) sc[t] = ref_expf_det(sc[t] - M);
                    tree[j] = t < n_kv ? (double) sc[t] : 0.0;
                }
                for (int64_t w = 1; w < C; w <<= 1)
                    for (int64_t j = 0; j < C; j += 2 * w) tree[j] = tree[j] + tree[j + w];
                sum += tree[0];
            }
            const float inv = (float) (1.0 / sum);
            float acc[512];
            for (int64_t d = 0; d < D; d++) acc[d] = 0.0f;
            for (int64_t t = 0; t < n_kv; t++) {
                float p = sc[t] * inv;
                if (!prec_f32) p = ref_fp16_to_fp32(ref_fp32_to_fp16(p));
                if (p == 0.0f) continue;
                const uint16_t * vr = vb + t * kv_stride_pos;
                const __m256 p8 = _mm256_set1_ps(p);
                for (int64_t d = 0; d < D; d += 8) {
                    const __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (vr + d)));
                    _mm256_storeu_ps(acc + d, _mm256_fmadd_ps(p8, vf, _mm256_loadu_ps(acc + d)));
                }
            }
            float * o = out + (iq * Hq + h) * D;
            for (int64_t d = 0; d < D; d++) o[d] = acc[d];
            free(sc);
        }
    }
}

/* ggml_compute_forward_flash_attn_ext_f16_one_chunk restated: sequential
 * online softmax over KV positions, masked (-inf) positions skipped. */
void ref_flash_attn_ext(const float * q, int64_t q_stride_tok, int64_t q_stride_head,
                        const uint16_t * k, const uint16_t * v, int64_t kv_stride_head,
                        int64_t kv_stride_pos, const uint16_t * mask, int64_t mask_stride,
                        float * out, int64_t D, int64_t n_q, int64_t Hq, int64_t Hkv, int64_t n_kv,
                        float scale, int fidelity, int n_threads) {
    const int64_t group = Hq / Hkv;
    if (fidelity == 6 || fidelity == 7) {
        /* the unfused chain in place of the fused op (6: GGML_PREC_F32) */
        ref_naive_attention(q, q_stride_tok, q_stride_head, k, v, kv_stride_head, kv_stride_pos, mask, mask_stride,
                            out, D, n_q, Hq, Hkv, n_kv, scale, fidelity == 6, n_threads);
        return;
    }
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
#else
    (void) n_threads;
#endif
#pragma omp parallel for collapse(2) num_threads(n_threads) schedule(static)
    for (int64_t iq = 0; iq < n_q; iq++) {
        for (int64_t h = 0; h < Hq; h++) {
            const int64_t kvh = h / group;
            const float * qr = q + iq * q_stride_tok + h * q_stride_head;
            uint16_t qh[512];
            float qf[512];
            uint16_t acc16[512];
            float acc32[512];
            for (int64_t d = 0; d < D; d++) {
                qh[d] = ref_fp32_to_fp16(qr[d]);
                qf[d] = qr[d];
                acc16[d] = 0;
                acc32[d] = 0.0f;
            }
            float * o = out + (iq * Hq + h) * D;
            if (fidelity == 5) {
                fa_chunked5_one(qh, k + kvh * kv_stride_head, v + kvh * kv_stride_head, kv_stride_pos,
                                mask ? mask + iq * mask_stride : NULL, o, D, n_kv, scale);
                continue;
            }
            if (fidelity == 4) {
                fa_chunked_one(qh, k + kvh * kv_stride_head, v + kvh * kv_stride_head, kv_stride_pos,
                               mask ? mask + iq * mask_stride : NULL, o, D, n_kv, scale);
                continue;
            }
            if (fidelity == 3) {
                /* two-pass: global max first, then every p = exp(s - M) and the
                 * sums in f64, one rounding at the end */
                float M = -INFINITY;
                for (int64_t ic = 0; ic < n_kv; ic++) {
                    const float mv = mask ? ref_fp16_to_fp32(mask[iq * mask_stride + ic]) : 0.0f;
                    if (mv == -INFINITY) continue;
                    const uint16_t * kr = k + kvh * kv_stride_head + ic * kv_stride_pos;
                    double a = 0.0;
                    for (int64_t d = 0; d < D; d++) a += (double) (ref_fp16_to_fp32(kr[d]) * ref_fp16_to_fp32(qh[d]));
                    const float s = (float) a * scale + mv;
                    M = s > M ? s : M;
                }
                double l = 0.0;
                double acc[512];
                for (int64_t d = 0; d < D; d++) acc[d] = 0.0;
                if (M != -INFINITY) {
                    for (int64_t ic = 0; ic < n_kv; ic++) {
                        const float mv = mask ? ref_fp16_to_fp32(mask[iq * mask_stride + ic]) : 0.0f;
                        if (mv == -INFINITY) continue;
                        const uint16_t * kr = k + kvh * kv_stride_head + ic * kv_stride_pos;
                        const uint16_t * vr = v + kvh * kv_stride_head + ic * kv_stride_pos;
                        double a = 0.0;
                        for (int64_t d = 0; d < D; d++) a += (double) (ref_fp16_to_fp32(kr[d]) * ref_fp16_to_fp32(qh[d]));
                        const float s = (float) a * scale + mv;
                        const float p = ref_expf_det(s - M);
                        l += (double) p;
                        for (int64_t d = 0; d < D; d++) acc[d] += (double) p * (double) ref_fp16_to_fp32(vr[d]);
                    }
                }
                for (int64_t d = 0; d < D; d++) o[d] = l == 0.0 ? 0.0f : (float) (acc[d] / l);
                continue;
            }
            float M = -INFINITY, S = 0.0f;
            for (int64_t ic = 0; ic < n_kv; ic++) {
                const float mv = mask ? ref_fp16_to_fp32(mask[iq * mask_stride + ic]) : 0.0f;
                if (mv == -INFINITY) continue;
                const uint16_t * kr = k + kvh * kv_stride_head + ic * kv_stride_pos;
                const uint16_t * vr = v + kvh * kv_stride_head + ic * kv_stride_pos;
                float s;
                if (fidelity == 1) {
                    s = ref_vec_dot_f16(D, kr, qh);
                } else if (fidelity == 2) {
                    double a = 0.0;
                    for (int64_t d = 0; d < D; d++) a += (double) ref_fp16_to_fp32(kr[d]) * ref_fp16_to_fp32(qh[d]);
                    s = (float) a;
                } else {
                    double a = 0.0;
                    for (int64_t d = 0; d < D; d++) a += (double) ref_fp16_to_fp32(kr[d]) * qf[d];
                    s = (float) a;
                }
                s = s * scale + mv;
                const float Mold = M;
                float ms = 1.0f, vs = 1.0f;
                if (s > M) {
                    M = s;
                    ms = ref_expf_det(Mold - M);
                    for (int64_t d = 0; d < D; d++) {
                        if (fidelity == 1) acc16[d] = ref_fp32_to_fp16(ref_fp16_to_fp32(acc16[d]) * ms);
                        else acc32[d] *= ms;
                    }
                } else {
                    vs = ref_expf_det(s - M);
                }
                for (int64_t d = 0; d < D; d++) {
                    if (fidelity == 1) {
                        acc16[d] = ref_fp32_to_fp16(fmaf(ref_fp16_to_fp32(vr[d]), vs, ref_fp16_to_fp32(acc16[d])));
                    } else {
                        acc32[d] += ref_fp16_to_fp32(vr[d]) * vs;
                    }
                }
                S = S * ms + vs;
            }
            const float inv = S == 0.0f ? 0.0f : 1.0f / S;
            for (int64_t d = 0; d < D; d++) o[d] = (fidelity == 1 ? ref_fp16_to_fp32(acc16[d]) : acc32[d]) * inv;
        }
    }
}
