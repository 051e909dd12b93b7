/*
 * ggml_cpu_ref.h -- CPU restatement of the ggml-cpu semantics on OpenASR's
 * quantized decoder path. TEST INFRASTRUCTURE ONLY: the parity tests, the
 * smoke check and the benchmark's CPU-baseline leg call it as the checker;
 * nothing in the product links it.
 *
 * The arithmetic of the reference path lives in the un-vendored openasr-ggml
 * fork (crates/openasr-core/third_party/openasr-ggml, pinned at
 * 0db3a287511085fb1564fea3f86839f9e40ca39e per
 * model-registry/catalog.public.json:3941), which is absent here. Every
 * function below restates ggml's published algorithm for the op named in its
 * comment and cites the reference call site that reaches it.
 *
 * Parity status per function (pinned = checked by known-answer tests, closed
 * forms, brute force or invariants in tests/test_oracle.py):
 *   fp16 conversion, Q8_0/Q4_K/Q8_K block codecs, vec_dot_q8_0_q8_0,
 *   vec_dot_q4_K_q8_K, mul_mat, rms_norm, norm, rope_neox, silu, gelu,
 *   soft_max_ext, flash_attn_ext, argmax, set_rows, get_rows: pinned.
 *   The float accumulation ORDER inside ggml-cpu's SIMD dot products and its
 *   vectorised expf are ISA-specific and cannot be pinned without the fork;
 *   this restatement accumulates in a fixed scalar order (parity unpinned at
 *   the ulp level only).
 */
#ifndef OPENASR_ORACLE_GGML_CPU_REF_H
#define OPENASR_ORACLE_GGML_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define REF_QK8_0 32
#define REF_QK_K 256

/* ggml block layouts (ggml-common.h) */
typedef struct {
    uint16_t d;
    int8_t qs[REF_QK8_0];
} ref_block_q8_0; /* 34 bytes */

typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[REF_QK_K / 2];
} ref_block_q4_K; /* 144 bytes */

typedef struct {
    uint8_t hmask[REF_QK_K / 8]; /* third bit of each quant, clear = minus 4 */
    uint8_t qs[REF_QK_K / 4];    /* two low bits of each quant */
    uint8_t scales[12];          /* sixteen 6-bit scales, stored minus 32 */
    uint16_t d;
} ref_block_q3_K; /* 110 bytes */

typedef struct {
    float d;
    int8_t qs[REF_QK_K];
    int16_t bsums[REF_QK_K / 16];
} ref_block_q8_K; /* 292 bytes */

/* element-type codes, as ggml numbers them */
enum { REF_F32 = 0, REF_F16 = 1, REF_Q8_0 = 8, REF_Q3_K = 11, REF_Q4_K = 12, REF_Q8_K = 15 };

uint16_t ref_fp32_to_fp16(float f);
float ref_fp16_to_fp32(uint16_t h);
void ref_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n);
void ref_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n);

/* weight quantizers (ggml_quantize_chunk, gguf_write.rs:579-588) */
void ref_quantize_row_q8_0_weights(const float * x, ref_block_q8_0 * y, int64_t k);
void ref_quantize_row_q4_K(const float * x, ref_block_q4_K * y, int64_t k);
/* activation quantizers (ggml-cpu from_float for the vec_dot_type) */
void ref_quantize_row_q8_0_act(const float * x, ref_block_q8_0 * y, int64_t k);
void ref_quantize_row_q8_K(const float * x, ref_block_q8_K * y, int64_t k);

void ref_dequantize_row_q8_0(const ref_block_q8_0 * x, float * y, int64_t k);
void ref_dequantize_row_q4_K(const ref_block_q4_K * x, float * y, int64_t k);
void ref_dequantize_row_q3_K(const ref_block_q3_K * x, float * y, int64_t k);
int ref_q3_K_scale(const uint8_t * scales, int i);
void ref_dequantize_row_q8_K(const ref_block_q8_K * x, float * y, int64_t k);
void ref_get_scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m);

float ref_vec_dot_q8_0_q8_0(int64_t n, const ref_block_q8_0 * x, const ref_block_q8_0 * y);
float ref_vec_dot_q4_K_q8_K(int64_t n, const ref_block_q4_K * x, const ref_block_q8_K * y);
float ref_vec_dot_q3_K_q8_K(int64_t n, const ref_block_q3_K * x, const ref_block_q8_K * y);
float ref_vec_dot_f16(int64_t n, const uint16_t * x, const uint16_t * y);

size_t ref_row_size(int type, int64_t ne0);

/*
 * GGML_OP_MUL_MAT (cpu_graph.rs:3652-3686): dst[n][m] = dot(W row m, x col n)
 * with x converted to W's vec_dot type first. W rows are contiguous with
 * stride row_bytes; x is f32 [n][k] with row stride x_stride floats; dst is
 * f32 [n][m] with stride d_stride floats.
 */
void ref_mul_mat(int wtype, const void * w, size_t row_bytes, int64_t m, int64_t k,
                 const float * x, int64_t x_stride, int64_t n, float * dst, int64_t d_stride,
                 int n_threads);

/* elementwise / row ops (ggml-cpu ops.cpp restated) */
void ref_rms_norm(const float * x, float * y, int64_t ne0, int64_t rows, float eps);
void ref_norm(const float * x, float * y, int64_t ne0, int64_t rows, float eps);
float ref_silu(float x);
float ref_gelu_f32(float x); /* closed-form tanh approximation */
float ref_gelu(float x);     /* ggml-cpu: through the f16 lookup table */
void ref_rope_neox(const float * x, float * y, int64_t head_dim, int64_t n_heads, int64_t n_tokens,
                   const int32_t * pos, int n_dims, float freq_base, float freq_scale);
void ref_soft_max_ext(const float * x, const uint16_t * mask, float * y, int64_t ne0, int64_t rows,
                      float scale);
int32_t ref_argmax_last(const float * x, int64_t n);
float ref_expf_det(float x);
float ref_erff_det(float x);
double ref_erf_coef(int n); /* coefficient a_n (n < 64) of ref_erff_det's series */
float ref_gelu_erf(float x); /* 0.5 x (1 + erf(x / sqrt 2)), erf by ref_erff_det */
float ref_relu(float x);
void ref_sincosf_det(float x, float * s_out, float * c_out);
int32_t ref_argmax_first(const float * x, int64_t n);

/*
 * GGML_OP_FLASH_ATTN_EXT (cpu_graph.rs:4144-4215) for one sequence:
 *   q    f32 [n_q][Hq][D] addressed by (q_stride_tok, q_stride_head) floats
 *   k,v  f16 [Hkv][n_kv][D] addressed by (kv_stride_head, kv_stride_pos) halves
 *   mask f16 [n_q][n_kv] (row stride mask_stride) or NULL
 *   out  f32 [n_q][Hq][D] contiguous
 * q head h reads kv head h / (Hq / Hkv). fidelity=1 reproduces ggml-cpu's
 * f16-rounded Q and f16 V accumulator; fidelity=2 rounds Q to f16 but
 * accumulates V in f32; fidelity=0 keeps Q in f32 and accumulates in f32;
 * fidelity=3 rounds Q to f16, takes the global max first and accumulates
 * p = exp(s - max), the sum and p*V in f64, rounding once.
 * fidelity=4 rounds Q to f16 and splits the span into fixed 64-position
 * chunks: per chunk the max m_c, p = exp(s - m_c) and the f64 sums
 * l_c = sum p, a_c = sum p*V; then M = max m_c and, in chunk order,
 * w = exp(m_c - M), L += w*l_c, O += w*a_c; out = O/L rounded once.
 * fidelity=5 (the device's definition) has the chunks of fidelity 4 with
 * f32 arithmetic in a fixed order inside a chunk: each score is the f32 fma
 * chain over dims in order (times scale, plus the mask value), l_c = l_c + p
 * and a_c = fma(p, V, a_c) in f32 over the chunk's live positions in order;
 * the chunk combine is fidelity 4's, in f64.
 * fidelity=6 and 7 compute the unfused chain the host emits in its place
 * (ref_naive_attention; 6 with GGML_PREC_F32 on its products, 7 without).
 */
void ref_flash_attn_ext(const float * q, int64_t q_stride_tok, int64_t q_stride_head,
                        const uint16_t * k, const uint16_t * v, int64_t kv_stride_head,
                        int64_t kv_stride_pos, const uint16_t * mask, int64_t mask_stride,
                        float * out, int64_t D, int64_t n_q, int64_t Hq, int64_t Hkv, int64_t n_kv,
                        float scale, int fidelity, int n_threads);

/*
 * llm_naive_masked_attention (nn/decoder.rs:2154-2200): MUL_MAT(K, Q) ->
 * SOFT_MAX_EXT(mask, scale) -> MUL_MAT(CONT(V^T), P) -> PERMUTE/CONT, same
 * layouts as ref_flash_attn_ext; prec_f32: GGML_PREC_F32 on both products
 * (Q and P kept f32), else Q and P rounded to f16. The order of every sum is
 * fixed (see the definition in ggml_cpu_ref.c).
 */
void ref_naive_attention(const float * q, int64_t q_stride_tok, int64_t q_stride_head, const uint16_t * k,
                         const uint16_t * v, int64_t kv_stride_head, int64_t kv_stride_pos, const uint16_t * mask,
                         int64_t mask_stride, float * out, int64_t D, int64_t n_q, int64_t Hq, int64_t Hkv,
                         int64_t n_kv, float scale, int prec_f32, int n_threads);

#ifdef __cplusplus
}
#endif

#endif
