/*
 * cpu_fast.c -- the CPU baseline leg of the benchmark: the batched Qwen3
 * decode step with ggml-cpu's arithmetic classes on the host ISA. TEST AND
 * MEASUREMENT INFRASTRUCTURE ONLY: bench.py times it beside the device as
 * the "ggml-cpu-class restatement"; tests/test_cpu_fast.py checks it
 * against the oracle (ggml_cpu_ref.c, ref_decoder.c), which stays the
 * checker. Nothing in the product links it.
 *
 * What it restates of ggml-cpu (the fork's ggml-cpu is absent, see
 * ggml_cpu_ref.h; the published algorithms are followed):
 *   - activations quantized to the weight's vec_dot type (Q8_K for Q4_K,
 *     Q8_0 for Q8_0) once per MUL_MAT, as ggml_compute_forward_mul_mat does;
 *   - ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q8_0_q8_0: integer dots of each
 *     block in SIMD registers (AVX-512 VNNI dpbusd where the CPU has it,
 *     AVX2 maddubs otherwise), each block's integer sum scaled and added into
 *     f32 vector accumulators with fma (not the oracle's f64 block sums);
 *   - the rows of a MUL_MAT split over the threads, every column of a row
 *     block computed while its weights are in cache;
 *   - flash attention for one query: ggml_vec_dot_f16 scores (f16 query,
 *     f32 SIMD accumulation), online softmax, V accumulated in f16
 *     (ggml_vec_mad_f16 / ggml_vec_scale_f16), one (sequence, head) a task;
 *   - norms, RoPE, SiLU and the first-max argmax as the oracle has them
 *     (they are a vanishing share of the step).
 * The op sequence is the oracle's ref_qwen_decode_batch (the decoder layer
 * of crates/openasr-core/src/nn/decoder.rs:1850-2145 over n_seq sequences).
 */
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "ggml_cpu_ref.h"

/* ----------------------------------------------------------- dot kernels -- */

static float hsum256(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* the eight 6-bit scales and mins of a Q4_K super-block (the packing
 * ref_get_scale_min_k4 reads: j < 4 in the low six bits of bytes j and
 * j + 4, j >= 4 split over the low / high nibble of byte j + 4 and the top
 * two bits of bytes j - 4 and j), decoded inline */
static inline void q4k_scales(const uint8_t * q, uint8_t * s8, uint8_t * m8) {
    for (int j = 0; j < 4; j++) {
        s8[j] = q[j] & 63;
        m8[j] = q[j + 4] & 63;
        s8[j + 4] = (uint8_t) ((q[j + 8] & 0xF) | ((q[j] >> 6) << 4));
        m8[j + 4] = (uint8_t) ((q[j + 8] >> 4) | ((q[j + 4] >> 6) << 4));
    }
}

__attribute__((target("f16c"))) static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

/* ggml_vec_dot_q4_K_q8_K: per super-block d = y.d * x.d, dmin = y.d * x.dmin;
 * the integer sums of the eight 32-element sub-blocks times their 6-bit
 * scales, and the mins against the activations' 16-element sums; both added
 * into f32 vector accumulators. AVX2 form: maddubs of the 4-bit values with
 * the activations, madd by the sub-block scale. */
__attribute__((target("avx2,fma,f16c"))) static float dot_q4_K_avx2(int64_t nb, const ref_block_q4_K * x,
                                                                   const ref_block_q8_K * y) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    float acc_m = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        const float d = y[i].d * h2f(x[i].d);
        const float dmin = -y[i].d * h2f(x[i].dmin);
        uint8_t s8[8], m8[8];
        q4k_scales(x[i].scales, s8, m8);
        int summ = 0;
        for (int j = 0; j < 8; j++) summ += m8[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        acc_m = fmaf(dmin, (float) summ, acc_m);
        __m256i sumi = _mm256_setzero_si256();
        const uint8_t * q4 = x[i].qs;
        const int8_t * q8 = y[i].qs;
        for (int j = 0; j < 4; j++) {
            const __m256i bits = _mm256_loadu_si256((const __m256i *) q4);
            const __m256i lo = _mm256_and_si256(bits, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
            const __m256i y0 = _mm256_loadu_si256((const __m256i *) q8);
            const __m256i y1 = _mm256_loadu_si256((const __m256i *) (q8 + 32));
            const __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, y0), _mm256_set1_epi16(s8[2 * j]));
            const __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, y1), _mm256_set1_epi16(s8[2 * j + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
            q4 += 32;
            q8 += 64;
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum256(acc) + acc_m;
}

/* the same with VNNI: dpbusd of the 4-bit values (unsigned) and the
 * activations (signed) into int32 lanes, one accumulator a sub-block, then
 * the scale multiply */
__attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512bw,avx512vnni"))) static float dot_q4_K_vnni(
    int64_t nb, const ref_block_q4_K * x, const ref_block_q8_K * y) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    float acc_m = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        const float d = y[i].d * h2f(x[i].d);
        const float dmin = -y[i].d * h2f(x[i].dmin);
        uint8_t s8[8], m8[8];
        q4k_scales(x[i].scales, s8, m8);
        int summ = 0;
        for (int j = 0; j < 8; j++) summ += m8[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        acc_m = fmaf(dmin, (float) summ, acc_m);
        __m256i sumi = _mm256_setzero_si256();
        const uint8_t * q4 = x[i].qs;
        const int8_t * q8 = y[i].qs;
        for (int j = 0; j < 4; j++) {
            const __m256i bits = _mm256_loadu_si256((const __m256i *) q4);
            const __m256i lo = _mm256_and_si256(bits, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
            const __m256i d0 = _mm256_dpbusd_epi32(_mm256_setzero_si256(), lo, _mm256_loadu_si256((const __m256i *) q8));
            const __m256i d1 =
                _mm256_dpbusd_epi32(_mm256_setzero_si256(), hi, _mm256_loadu_si256((const __m256i *) (q8 + 32)));
            sumi = _mm256_add_epi32(sumi, _mm256_mullo_epi32(d0, _mm256_set1_epi32(s8[2 * j])));
            sumi = _mm256_add_epi32(sumi, _mm256_mullo_epi32(d1, _mm256_set1_epi32(s8[2 * j + 1])));
            q4 += 32;
            q8 += 64;
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum256(acc) + acc_m;
}

/* The Q4_K dot of one weight row with nc (<= 8) activation columns at once,
 * as ggml-cpu's repacked Q4_K GEMM reuses a decoded weight block across the
 * columns: each super-block's scales, mins and nibbles are decoded once, then
 * every column's integer sub-block sums (VNNI dpbusd) are scaled and added
 * into that column's f32 accumulators; the per-column arithmetic is the
 * single-column dot's. */
__attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512bw,avx512vnni"))) static void dot_q4_K_multi_vnni(
    int64_t nb, const ref_block_q4_K * x, const ref_block_q8_K * const * y, int nc, float * out) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc[8];
    float acc_m[8];
    for (int c = 0; c < nc; c++) {
        acc[c] = _mm256_setzero_ps();
        acc_m[c] = 0.0f;
    }
    for (int64_t i = 0; i < nb; i++) {
        uint8_t s8[8], m8[8];
        q4k_scales(x[i].scales, s8, m8);
        const float xd = h2f(x[i].d), xm = h2f(x[i].dmin);
        __m256i lo[4], hi[4];
        for (int j = 0; j < 4; j++) {
            const __m256i bits = _mm256_loadu_si256((const __m256i *) (x[i].qs + 32 * j));
            lo[j] = _mm256_and_si256(bits, m4);
            hi[j] = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
        }
        for (int c = 0; c < nc; c++) {
            const ref_block_q8_K * yc = y[c] + i;
            int summ = 0;
            for (int j = 0; j < 8; j++) summ += m8[j] * (yc->bsums[2 * j] + yc->bsums[2 * j + 1]);
            acc_m[c] = fmaf(-yc->d * xm, (float) summ, acc_m[c]);
            __m256i sumi = _mm256_setzero_si256();
            for (int j = 0; j < 4; j++) {
                const __m256i d0 =
                    _mm256_dpbusd_epi32(_mm256_setzero_si256(), lo[j], _mm256_loadu_si256((const __m256i *) (yc->qs + 64 * j)));
                const __m256i d1 = _mm256_dpbusd_epi32(_mm256_setzero_si256(), hi[j],
                                                       _mm256_loadu_si256((const __m256i *) (yc->qs + 64 * j + 32)));
                sumi = _mm256_add_epi32(sumi, _mm256_mullo_epi32(d0, _mm256_set1_epi32(s8[2 * j])));
                sumi = _mm256_add_epi32(sumi, _mm256_mullo_epi32(d1, _mm256_set1_epi32(s8[2 * j + 1])));
            }
            acc[c] = _mm256_fmadd_ps(_mm256_set1_ps(yc->d * xd), _mm256_cvtepi32_ps(sumi), acc[c]);
        }
    }
    for (int c = 0; c < nc; c++) out[c] = hsum256(acc[c]) + acc_m[c];
}

__attribute__((target("avx2,fma,f16c"))) static void dot_q4_K_multi_avx2(int64_t nb, const ref_block_q4_K * x,
                                                                        const ref_block_q8_K * const * y, int nc,
                                                                        float * out) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc[8];
    float acc_m[8];
    for (int c = 0; c < nc; c++) {
        acc[c] = _mm256_setzero_ps();
        acc_m[c] = 0.0f;
    }
    for (int64_t i = 0; i < nb; i++) {
        uint8_t s8[8], m8[8];
        q4k_scales(x[i].scales, s8, m8);
        const float xd = h2f(x[i].d), xm = h2f(x[i].dmin);
        __m256i lo[4], hi[4];
        for (int j = 0; j < 4; j++) {
            const __m256i bits = _mm256_loadu_si256((const __m256i *) (x[i].qs + 32 * j));
            lo[j] = _mm256_and_si256(bits, m4);
            hi[j] = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
        }
        for (int c = 0; c < nc; c++) {
            const ref_block_q8_K * yc = y[c] + i;
            int summ = 0;
            for (int j = 0; j < 8; j++) summ += m8[j] * (yc->bsums[2 * j] + yc->bsums[2 * j + 1]);
            acc_m[c] = fmaf(-yc->d * xm, (float) summ, acc_m[c]);
            __m256i sumi = _mm256_setzero_si256();
            for (int j = 0; j < 4; j++) {
                const __m256i y0 = _mm256_loadu_si256((const __m256i *) (yc->qs + 64 * j));
                const __m256i y1 = _mm256_loadu_si256((const __m256i *) (yc->qs + 64 * j + 32));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(lo[j], y0),
                                                                _mm256_set1_epi16(s8[2 * j])));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(hi[j], y1),
                                                                _mm256_set1_epi16(s8[2 * j + 1])));
            }
            acc[c] = _mm256_fmadd_ps(_mm256_set1_ps(yc->d * xd), _mm256_cvtepi32_ps(sumi), acc[c]);
        }
    }
    for (int c = 0; c < nc; c++) out[c] = hsum256(acc[c]) + acc_m[c];
}

/* ggml_vec_dot_q8_0_q8_0: per 32-element block the integer dot (sign trick:
 * |x| unsigned against y with x's sign) times x.d * y.d into f32 lanes */
__attribute__((target("avx2,fma,f16c"))) static float dot_q8_0_avx2(int64_t nb, const ref_block_q8_0 * x,
                                                                   const ref_block_q8_0 * y) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int64_t i = 0; i < nb; i++) {
        const __m256i qx = _mm256_loadu_si256((const __m256i *) x[i].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *) y[i].qs);
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i s = _mm256_madd_epi16(_mm256_maddubs_epi16(ax, sy), ones);
        const float d = h2f(x[i].d) * h2f(y[i].d);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s), acc);
    }
    return hsum256(acc);
}

__attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512bw,avx512vnni"))) static float dot_q8_0_vnni(
    int64_t nb, const ref_block_q8_0 * x, const ref_block_q8_0 * y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < nb; i++) {
        const __m256i qx = _mm256_loadu_si256((const __m256i *) x[i].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *) y[i].qs);
        const __m256i s = _mm256_dpbusd_epi32(_mm256_setzero_si256(), _mm256_sign_epi8(qx, qx), _mm256_sign_epi8(qy, qx));
        const float d = h2f(x[i].d) * h2f(y[i].d);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s), acc);
    }
    return hsum256(acc);
}

static int have_vnni(void) {
    static int v = -1;
    if (v < 0) {
        __builtin_cpu_init();
        v = __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl") &&
            __builtin_cpu_supports("avx512bw");
    }
    return v;
}

int fast_cpu_uses_vnni(void) { return have_vnni(); }

float fast_vec_dot_q4_K_q8_K(int64_t n, const ref_block_q4_K * x, const ref_block_q8_K * y) {
    return have_vnni() ? dot_q4_K_vnni(n / REF_QK_K, x, y) : dot_q4_K_avx2(n / REF_QK_K, x, y);
}

float fast_vec_dot_q8_0_q8_0(int64_t n, const ref_block_q8_0 * x, const ref_block_q8_0 * y) {
    return have_vnni() ? dot_q8_0_vnni(n / REF_QK8_0, x, y) : dot_q8_0_avx2(n / REF_QK8_0, x, y);
}

/* ------------------------------------------------------------- mul_mat -- */

/* dst[n][m] = W row m . x column n: x quantized to the vec_dot type once,
 * rows in blocks of 16 over the threads, every column of a block while its
 * weights are in cache */
void fast_mul_mat(int wtype, const void * w, size_t row_bytes, int64_t m, int64_t k, const float * x,
                  int64_t x_stride, int64_t n, float * dst, int64_t d_stride, int n_threads) {
    const size_t qrow = wtype == REF_Q4_K ? (size_t) (k / REF_QK_K) * sizeof(ref_block_q8_K)
                                          : (size_t) (k / REF_QK8_0) * sizeof(ref_block_q8_0);
    char * xq = (char *) malloc(qrow * (size_t) n);
    for (int64_t j = 0; j < n; j++) {
        if (wtype == REF_Q4_K) ref_quantize_row_q8_K(x + j * x_stride, (ref_block_q8_K *) (xq + j * qrow), k);
        else ref_quantize_row_q8_0_act(x + j * x_stride, (ref_block_q8_0 *) (xq + j * qrow), k);
    }
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
#else
    (void) n_threads;
#endif
    const int64_t blk = 16, nblk = (m + blk - 1) / blk;
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t b = 0; b < nblk; b++) {
        const int64_t r1 = (b + 1) * blk < m ? (b + 1) * blk : m;
        if (wtype == REF_Q4_K) {
            // columns in groups of up to eight against each decoded weight row
            for (int64_t j0 = 0; j0 < n; j0 += 8) {
                const int nc = n - j0 < 8 ? (int) (n - j0) : 8;
                const ref_block_q8_K * ys[8];
                for (int c = 0; c < nc; c++) ys[c] = (const ref_block_q8_K *) (xq + (j0 + c) * qrow);
                for (int64_t r = b * blk; r < r1; r++) {
                    float o[8];
                    const ref_block_q4_K * wr = (const ref_block_q4_K *) ((const char *) w + (size_t) r * row_bytes);
                    if (have_vnni()) dot_q4_K_multi_vnni(k / REF_QK_K, wr, ys, nc, o);
                    else dot_q4_K_multi_avx2(k / REF_QK_K, wr, ys, nc, o);
                    for (int c = 0; c < nc; c++) dst[(j0 + c) * d_stride + r] = o[c];
                }
            }
            continue;
        }
        for (int64_t j = 0; j < n; j++) {
            for (int64_t r = b * blk; r < r1; r++) {
                const void * wr = (const char *) w + (size_t) r * row_bytes;
                dst[j * d_stride + r] =
                    wtype == REF_Q4_K
                        ? fast_vec_dot_q4_K_q8_K(k, (const ref_block_q4_K *) wr, (const ref_block_q8_K *) (xq + j * qrow))
                        : fast_vec_dot_q8_0_q8_0(k, (const ref_block_q8_0 *) wr, (const ref_block_q8_0 *) (xq + j * qrow));
            }
        }
    }
    free(xq);
}

/* --------------------------------------------------------- attention ----- */

/* ggml_vec_dot_f16 over D (a multiple of 32): four f32 accumulators of eight
 * lanes, then their sum */
__attribute__((target("avx2,fma,f16c"))) static float dot_f16(int64_t D, const uint16_t * a, const uint16_t * b) {
    __m256 s[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (int64_t d = 0; d < D; d += 32) {
        for (int u = 0; u < 4; u++) {
            const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (a + d + 8 * u)));
            const __m256 y = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (b + d + 8 * u)));
            s[u] = _mm256_fmadd_ps(x, y, s[u]);
        }
    }
    return hsum256(_mm256_add_ps(_mm256_add_ps(s[0], s[1]), _mm256_add_ps(s[2], s[3])));
}

/* one query row against an f16 K/V span of n_kv positions with an additive
 * f16 mask: the online softmax of ggml-cpu's flash attention with its f16 V
 * accumulator; out = VKQ / S */
__attribute__((target("avx2,fma,f16c"))) static void fa_one(const float * q, const uint16_t * k, const uint16_t * v,
                                                           int64_t pos_stride, const uint16_t * mask, int64_t n_kv,
                                                           int64_t D, float scale, float * out) {
    uint16_t qh[512], acc[512];
    for (int64_t d = 0; d < D; d++) {
        qh[d] = ref_fp32_to_fp16(q[d]);
        acc[d] = 0;
    }
    float M = -INFINITY, S = 0.0f;
    for (int64_t t = 0; t < n_kv; t++) {
        const float mv = mask ? ref_fp16_to_fp32(mask[t]) : 0.0f;
        if (mv == -INFINITY) continue;
        const float s = dot_f16(D, k + t * pos_stride, qh) * scale + mv;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            const float Mold = M;
            M = s;
            ms = expf(Mold - M);
            const __m256 m8 = _mm256_set1_ps(ms);
            for (int64_t d = 0; d < D; d += 8) {
                const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (acc + d)));
                _mm_storeu_si128((__m128i *) (acc + d), _mm256_cvtps_ph(_mm256_mul_ps(a, m8), _MM_FROUND_TO_NEAREST_INT));
            }
        } else {
            vs = expf(s - M);
        }
        const __m256 v8 = _mm256_set1_ps(vs);
        const uint16_t * vr = v + t * pos_stride;
        for (int64_t d = 0; d < D; d += 8) {
            const __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (acc + d)));
            const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (vr + d)));
            _mm_storeu_si128((__m128i *) (acc + d), _mm256_cvtps_ph(_mm256_fmadd_ps(x, v8, a), _MM_FROUND_TO_NEAREST_INT));
        }
        S = S * ms + vs;
    }
    const float inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int64_t d = 0; d < D; d++) out[d] = ref_fp16_to_fp32(acc[d]) * inv;
}

/* one query row (f32 [D]) against f16 K/V rows [n_kv][D] with an optional f16
 * mask: the attention of the decode step, for tests */
void fast_attn_one(const float * q, const uint16_t * k, const uint16_t * v, const uint16_t * mask, int64_t n_kv,
                   int64_t D, float scale, float * out) {
    fa_one(q, k, v, D, mask, n_kv, D, scale, out);
}

/* ------------------------------------------------------- decode step ----- */

typedef struct {
    int d_model, n_layers, n_head, n_kv_head, head_dim, ffn, vocab, wtype;
    float rope_theta, rms_eps;
    int out_wtype;
} fast_qwen_dims; /* the oracle's ref_qwen_dims */

enum { F_EMBD = 0, F_OUT_NORM = 1, F_LAYER0 = 2, F_PER_LAYER = 9 };

static const void * fp(const void * const * t, int layer, int idx) { return t[F_LAYER0 + layer * F_PER_LAYER + idx]; }

static void mul_w(float * x, const float * w, int rows, int n) {
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) x[(size_t) r * n + i] *= w[i];
}

void ref_qwen_embed(const fast_qwen_dims * m, const void * const * t, const int32_t * tokens, int T, float * out);

/* One decode step of n_seq sequences (ref_qwen_decode_batch's op sequence):
 * the projections as one MUL_MAT over the n_seq columns, attention per
 * (sequence, head) over its own cache. kcache/vcache: [seq * n_layers + layer]
 * f16 [n_kv_head][max_pos][head_dim]; pos[s] the position written this step.
 * top1 [n_seq] and logits [n_seq][vocab] (optional) out. */
void fast_qwen_decode_batch(const fast_qwen_dims * m, const void * const * t, uint16_t * const * kcache,
                            uint16_t * const * vcache, int max_pos, const int32_t * tokens, const int32_t * pos,
                            int n_seq, int32_t * top1, float * logits, int threads) {
    const int d = m->d_model, hd = m->head_dim, hq = m->n_head, hkv = m->n_kv_head, N = n_seq;
    const int q_w = hq * hd, kv_w = hkv * hd, qkv_w = q_w + 2 * kv_w, g = hq / hkv;
    const size_t rs_d = ref_row_size(m->wtype, d);
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#endif
    float * x = (float *) malloc(sizeof(float) * (size_t) N * d);
    float * nrm = (float *) malloc(sizeof(float) * (size_t) N * (d > m->ffn ? d : m->ffn));
    float * qkv = (float *) malloc(sizeof(float) * (size_t) N * qkv_w);
    float * q = (float *) malloc(sizeof(float) * (size_t) N * q_w);
    float * k = (float *) malloc(sizeof(float) * (size_t) N * kv_w);
    float * att = (float *) malloc(sizeof(float) * (size_t) N * q_w);
    float * tmp = (float *) malloc(sizeof(float) * (size_t) N * d);
    float * gt = (float *) malloc(sizeof(float) * (size_t) N * m->ffn);
    float * up = (float *) malloc(sizeof(float) * (size_t) N * m->ffn);
    float * lg = (float *) malloc(sizeof(float) * (size_t) N * m->vocab);
    uint16_t * mask = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) max_pos);
    for (int j = 0; j < max_pos; j++) mask[j] = 0;
    ref_qwen_embed(m, t, tokens, N, x);
    for (int l = 0; l < m->n_layers; l++) {
        ref_rms_norm(x, nrm, d, N, m->rms_eps);
        mul_w(nrm, (const float *) fp(t, l, 0), N, d);
        fast_mul_mat(m->wtype, fp(t, l, 1), rs_d, qkv_w, d, nrm, d, N, qkv, qkv_w, threads);
        for (int i = 0; i < N; i++) {
            memcpy(q + (size_t) i * q_w, qkv + (size_t) i * qkv_w, sizeof(float) * q_w);
            memcpy(k + (size_t) i * kv_w, qkv + (size_t) i * qkv_w + q_w, sizeof(float) * kv_w);
        }
        ref_rms_norm(q, q, hd, (int64_t) N * hq, m->rms_eps);
        mul_w(q, (const float *) fp(t, l, 2), N * hq, hd);
        ref_rms_norm(k, k, hd, (int64_t) N * hkv, m->rms_eps);
        mul_w(k, (const float *) fp(t, l, 3), N * hkv, hd);
        ref_rope_neox(q, q, hd, hq, N, pos, hd, m->rope_theta, 1.0f);
        ref_rope_neox(k, k, hd, hkv, N, pos, hd, m->rope_theta, 1.0f);
        for (int i = 0; i < N; i++) {
            uint16_t * kc = kcache[(size_t) i * m->n_layers + l];
            uint16_t * vc = vcache[(size_t) i * m->n_layers + l];
            for (int h = 0; h < hkv; h++) {
                ref_fp32_to_fp16_row(k + ((size_t) i * hkv + h) * hd, kc + ((size_t) h * max_pos + pos[i]) * hd, hd);
                ref_fp32_to_fp16_row(qkv + (size_t) i * qkv_w + q_w + kv_w + (size_t) h * hd,
                                     vc + ((size_t) h * max_pos + pos[i]) * hd, hd);
            }
        }
#pragma omp parallel for collapse(2) num_threads(threads) schedule(dynamic, 1)
        for (int i = 0; i < N; i++) {
            for (int h = 0; h < hq; h++) {
                const uint16_t * kc = kcache[(size_t) i * m->n_layers + l] + (size_t) (h / g) * max_pos * hd;
                const uint16_t * vc = vcache[(size_t) i * m->n_layers + l] + (size_t) (h / g) * max_pos * hd;
                fa_one(q + ((size_t) i * hq + h) * hd, kc, vc, hd, mask, pos[i] + 1, hd, 1.0f / sqrtf((float) hd),
                       att + ((size_t) i * hq + h) * hd);
            }
        }
        fast_mul_mat(m->wtype, fp(t, l, 4), ref_row_size(m->wtype, q_w), d, q_w, att, q_w, N, tmp, d, threads);
        for (size_t i = 0; i < (size_t) N * d; i++) x[i] = x[i] + tmp[i];
        ref_rms_norm(x, nrm, d, N, m->rms_eps);
        mul_w(nrm, (const float *) fp(t, l, 5), N, d);
        fast_mul_mat(m->wtype, fp(t, l, 6), rs_d, m->ffn, d, nrm, d, N, gt, m->ffn, threads);
        fast_mul_mat(m->wtype, fp(t, l, 7), rs_d, m->ffn, d, nrm, d, N, up, m->ffn, threads);
        for (size_t i = 0; i < (size_t) N * m->ffn; i++) gt[i] = ref_silu(gt[i]) * up[i];
        fast_mul_mat(m->wtype, fp(t, l, 8), ref_row_size(m->wtype, m->ffn), d, m->ffn, gt, m->ffn, N, tmp, d,
                     threads);
        for (size_t i = 0; i < (size_t) N * d; i++) x[i] = tmp[i] + x[i];
    }
    ref_rms_norm(x, nrm, d, N, m->rms_eps);
    mul_w(nrm, (const float *) t[F_OUT_NORM], N, d);
    const void * ow = t[F_LAYER0 + m->n_layers * F_PER_LAYER];
    const int lt = ow ? m->out_wtype : m->wtype;
    fast_mul_mat(lt, ow ? ow : t[F_EMBD], ref_row_size(lt, d), m->vocab, d, nrm, d, N, lg, m->vocab, threads);
    for (int i = 0; i < N; i++) top1[i] = ref_argmax_first(lg + (size_t) i * m->vocab, m->vocab);
    if (logits) memcpy(logits, lg, sizeof(float) * (size_t) N * m->vocab);
    free(x);
    free(nrm);
    free(qkv);
    free(q);
    free(k);
    free(att);
    free(tmp);
    free(gt);
    free(up);
    free(lg);
    free(mask);
}
