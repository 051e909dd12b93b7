/*
 * ref_decoder.c -- CPU reference of the decoder steps, built from the
 * restated ggml-cpu ops in ggml_cpu_ref.c. TEST INFRASTRUCTURE ONLY: the
 * end-to-end parity tests and the benchmark's CPU-baseline leg run it as the
 * checker.
 *
 * Qwen3 LLM step: the op sequence of llm_layer
 * (crates/openasr-core/src/nn/decoder.rs:1850-2145) and the fused logits head
 * (models/qwen/llm_transformer.rs:2096-2115), one sequence at a time (the
 * reference's batched == serial invariant, nn/decoder.rs:3412-3520, makes the
 * per-sequence run the definition of the batched one).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "ggml_cpu_ref.h"

typedef struct {
    int d_model, n_layers, n_head, n_kv_head, head_dim, ffn, vocab, wtype;
    float rope_theta, rms_eps;
    int out_wtype; /* type of a separate output projection */
} ref_qwen_dims;

/* pointer table: [tok_embd, out_norm, then per layer attn_norm, qkv, q_norm,
 * k_norm, o, ffn_norm, gate, up, down, then the output projection or NULL
 * when it is tied to tok_embd] */
enum { T_EMBD = 0, T_OUT_NORM = 1, T_LAYER0 = 2, T_PER_LAYER = 9 };

/* the logits projection: a separate output.weight, else the tied embedding
 * (llm_transformer.rs:2096-2115) */
static const void * lm_head(const ref_qwen_dims * m, const void * const * t, int * type) {
    const void * o = t[T_LAYER0 + m->n_layers * T_PER_LAYER];
    *type = o ? m->out_wtype : m->wtype;
    return o ? o : t[T_EMBD];
}

static const void * tp(const void * const * t, int layer, int idx) { return t[T_LAYER0 + layer * T_PER_LAYER + idx]; }

static void mul_row_weight(float * x, const float * w, int rows, int n) {
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) x[(size_t) r * n + i] *= w[i];
}

/* get_rows on the token embedding, dequantizing (cpu_graph.rs:3688-3732) */
void ref_qwen_embed(const ref_qwen_dims * m, const void * const * t, const int32_t * tokens, int T, float * out) {
    const size_t rs = ref_row_size(m->wtype, m->d_model);
    for (int i = 0; i < T; i++) {
        const void * row = (const char *) t[T_EMBD] + (size_t) tokens[i] * rs;
        if (m->wtype == REF_Q8_0) ref_dequantize_row_q8_0((const ref_block_q8_0 *) row, out + (size_t) i * m->d_model, m->d_model);
        else ref_dequantize_row_q4_K((const ref_block_q4_K *) row, out + (size_t) i * m->d_model, m->d_model);
    }
}

/*
 * T positions p0..p0+T-1 of one sequence through every layer. x [T][d] is the
 * layer-0 input (embeddings or hidden prefix). kcache/vcache: per layer f16
 * [n_kv_head][max_pos][head_dim]. The last position's logits go to logits
 * ([vocab]) when non-null; returns the first-max top-1 of them (or -1).
 */
int32_t ref_qwen_forward(const ref_qwen_dims * m, const void * const * t, uint16_t * const * kcache,
                         uint16_t * const * vcache, int max_pos, const float * x_in, int T, int p0, float * logits,
                         int fa_fidelity, int threads) {
    const int d = m->d_model, hd = m->head_dim, hq = m->n_head, hkv = m->n_kv_head;
    const int q_w = hq * hd, kv_w = hkv * hd, qkv_w = q_w + 2 * kv_w;
    const size_t rs_d = ref_row_size(m->wtype, d);
    float * x = (float *) malloc(sizeof(float) * (size_t) T * d);
    float * nrm = (float *) malloc(sizeof(float) * (size_t) T * (d > m->ffn ? d : m->ffn));
    float * qkv = (float *) malloc(sizeof(float) * (size_t) T * qkv_w);
    float * q = (float *) malloc(sizeof(float) * (size_t) T * q_w);
    float * k = (float *) malloc(sizeof(float) * (size_t) T * kv_w);
    float * att = (float *) malloc(sizeof(float) * (size_t) T * q_w);
    float * tmp = (float *) malloc(sizeof(float) * (size_t) T * d);
    float * g = (float *) malloc(sizeof(float) * (size_t) T * m->ffn);
    float * u = (float *) malloc(sizeof(float) * (size_t) T * m->ffn);
    int32_t * pos = (int32_t *) malloc(sizeof(int32_t) * (size_t) T);
    const int n_kv = p0 + T;
    uint16_t * mask = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) T * n_kv);
    memcpy(x, x_in, sizeof(float) * (size_t) T * d);
    for (int i = 0; i < T; i++) {
        pos[i] = p0 + i;
        for (int j = 0; j < n_kv; j++) mask[(size_t) i * n_kv + j] = j <= p0 + i ? 0 : 0xFC00;
    }
    for (int l = 0; l < m->n_layers; l++) {
        /* attention block */
        ref_rms_norm(x, nrm, d, T, m->rms_eps);
        mul_row_weight(nrm, (const float *) tp(t, l, 0), T, d);
        ref_mul_mat(m->wtype, tp(t, l, 1), rs_d, qkv_w, d, nrm, d, T, qkv, qkv_w, threads);
        for (int i = 0; i < T; i++) {
            memcpy(q + (size_t) i * q_w, qkv + (size_t) i * qkv_w, sizeof(float) * q_w);
            memcpy(k + (size_t) i * kv_w, qkv + (size_t) i * qkv_w + q_w, sizeof(float) * kv_w);
        }
        ref_rms_norm(q, q, hd, (int64_t) T * hq, m->rms_eps);
        mul_row_weight(q, (const float *) tp(t, l, 2), T * hq, hd);
        ref_rms_norm(k, k, hd, (int64_t) T * hkv, m->rms_eps);
        mul_row_weight(k, (const float *) tp(t, l, 3), T * hkv, hd);
        ref_rope_neox(q, q, hd, hq, T, pos, hd, m->rope_theta, 1.0f);
        ref_rope_neox(k, k, hd, hkv, T, pos, hd, m->rope_theta, 1.0f);
        /* set_rows f32 -> f16 into the cache (nn/decoder.rs:2031-2036) */
        for (int i = 0; i < T; i++) {
            for (int h = 0; h < hkv; h++) {
                uint16_t * kd = kcache[l] + ((size_t) h * max_pos + pos[i]) * hd;
                uint16_t * vd = vcache[l] + ((size_t) h * max_pos + pos[i]) * hd;
                ref_fp32_to_fp16_row(k + ((size_t) i * hkv + h) * hd, kd, hd);
                ref_fp32_to_fp16_row(qkv + (size_t) i * qkv_w + q_w + kv_w + (size_t) h * hd, vd, hd);
            }
        }
        ref_flash_attn_ext(q, (int64_t) hq * hd, hd, kcache[l], vcache[l], (int64_t) max_pos * hd, hd, mask, n_kv,
                           att, hd, T, hq, hkv, n_kv, 1.0f / sqrtf((float) hd), fa_fidelity, threads);
        ref_mul_mat(m->wtype, tp(t, l, 4), ref_row_size(m->wtype, q_w), d, q_w, att, q_w, T, tmp, d, threads);
        for (size_t i = 0; i < (size_t) T * d; i++) x[i] = x[i] + tmp[i];
        /* SwiGLU block (nn/ffn.rs:64-91) */
        ref_rms_norm(x, nrm, d, T, m->rms_eps);
        mul_row_weight(nrm, (const float *) tp(t, l, 5), T, d);
        ref_mul_mat(m->wtype, tp(t, l, 6), rs_d, m->ffn, d, nrm, d, T, g, m->ffn, threads);
        ref_mul_mat(m->wtype, tp(t, l, 7), rs_d, m->ffn, d, nrm, d, T, u, m->ffn, threads);
        for (size_t i = 0; i < (size_t) T * m->ffn; i++) g[i] = ref_silu(g[i]) * u[i];
        ref_mul_mat(m->wtype, tp(t, l, 8), ref_row_size(m->wtype, m->ffn), d, m->ffn, g, m->ffn, T, tmp, d, threads);
        for (size_t i = 0; i < (size_t) T * d; i++) x[i] = tmp[i] + x[i];
    }
    int32_t top1 = -1;
    if (logits) {
        /* fused logits head on the last position (llm_transformer.rs:2096-2115) */
        float * last = x + (size_t) (T - 1) * d;
        ref_rms_norm(last, nrm, d, 1, m->rms_eps);
        mul_row_weight(nrm, (const float *) t[T_OUT_NORM], 1, d);
        int lt;
        const void * lw = lm_head(m, t, &lt);
        ref_mul_mat(lt, lw, ref_row_size(lt, d), m->vocab, d, nrm, d, 1, logits, m->vocab, threads);
        top1 = ref_argmax_first(logits, m->vocab);
    }
    free(x);
    free(nrm);
    free(qkv);
    free(q);
    free(k);
    free(att);
    free(tmp);
    free(g);
    free(u);
    free(pos);
    free(mask);
    return top1;
}

/*
 * One decode step of n_seq sequences at once (the serve-batch step,
 * models/qwen/batched_decode.rs:894-975): the projections run as one
 * mul_mat over n_seq columns (weights streamed once), attention per
 * sequence over its own cache. kcache/vcache: [seq * n_layers + layer].
 * top1 [n_seq] and logits [n_seq][vocab] (optional) out.
 */
void ref_qwen_decode_batch(const ref_qwen_dims * m, const void * const * t, uint16_t * const * kcache,
                           uint16_t * const * vcache, int max_pos, const int32_t * tokens, const int32_t * pos,
                           int n_seq, int32_t * top1, float * logits, int fa_fidelity, int threads) {
    const int d = m->d_model, hd = m->head_dim, hq = m->n_head, hkv = m->n_kv_head, N = n_seq;
    const int q_w = hq * hd, kv_w = hkv * hd, qkv_w = q_w + 2 * kv_w;
    const size_t rs_d = ref_row_size(m->wtype, d);
    float * x = (float *) malloc(sizeof(float) * (size_t) N * d);
    float * nrm = (float *) malloc(sizeof(float) * (size_t) N * (d > m->ffn ? d : m->ffn));
    float * qkv = (float *) malloc(sizeof(float) * (size_t) N * qkv_w);
    float * q = (float *) malloc(sizeof(float) * (size_t) N * q_w);
    float * k = (float *) malloc(sizeof(float) * (size_t) N * kv_w);
    float * att = (float *) malloc(sizeof(float) * (size_t) N * q_w);
    float * tmp = (float *) malloc(sizeof(float) * (size_t) N * d);
    float * g = (float *) malloc(sizeof(float) * (size_t) N * m->ffn);
    float * u = (float *) malloc(sizeof(float) * (size_t) N * m->ffn);
    float * lg = (float *) malloc(sizeof(float) * (size_t) N * m->vocab);
    uint16_t * mask = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) max_pos);
    ref_qwen_embed(m, t, tokens, N, x);
    for (int l = 0; l < m->n_layers; l++) {
        ref_rms_norm(x, nrm, d, N, m->rms_eps);
        mul_row_weight(nrm, (const float *) tp(t, l, 0), N, d);
        ref_mul_mat(m->wtype, tp(t, l, 1), rs_d, qkv_w, d, nrm, d, N, qkv, qkv_w, threads);
        for (int i = 0; i < N; i++) {
            memcpy(q + (size_t) i * q_w, qkv + (size_t) i * qkv_w, sizeof(float) * q_w);
            memcpy(k + (size_t) i * kv_w, qkv + (size_t) i * qkv_w + q_w, sizeof(float) * kv_w);
        }
        ref_rms_norm(q, q, hd, (int64_t) N * hq, m->rms_eps);
        mul_row_weight(q, (const float *) tp(t, l, 2), N * hq, hd);
        ref_rms_norm(k, k, hd, (int64_t) N * hkv, m->rms_eps);
        mul_row_weight(k, (const float *) tp(t, l, 3), N * hkv, hd);
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
            const int n_kv = pos[i] + 1;
            for (int j = 0; j < n_kv; j++) mask[j] = 0;
            ref_flash_attn_ext(q + (size_t) i * q_w, q_w, hd, kc, vc, (int64_t) max_pos * hd, hd, mask, n_kv,
                               att + (size_t) i * q_w, hd, 1, hq, hkv, n_kv, 1.0f / sqrtf((float) hd), fa_fidelity,
                               threads);
        }
        ref_mul_mat(m->wtype, tp(t, l, 4), ref_row_size(m->wtype, q_w), d, q_w, att, q_w, N, tmp, d, threads);
        for (size_t i = 0; i < (size_t) N * d; i++) x[i] = x[i] + tmp[i];
        ref_rms_norm(x, nrm, d, N, m->rms_eps);
        mul_row_weight(nrm, (const float *) tp(t, l, 5), N, d);
        ref_mul_mat(m->wtype, tp(t, l, 6), rs_d, m->ffn, d, nrm, d, N, g, m->ffn, threads);
        ref_mul_mat(m->wtype, tp(t, l, 7), rs_d, m->ffn, d, nrm, d, N, u, m->ffn, threads);
        for (size_t i = 0; i < (size_t) N * m->ffn; i++) g[i] = ref_silu(g[i]) * u[i];
        ref_mul_mat(m->wtype, tp(t, l, 8), ref_row_size(m->wtype, m->ffn), d, m->ffn, g, m->ffn, N, tmp, d, threads);
        for (size_t i = 0; i < (size_t) N * d; i++) x[i] = tmp[i] + x[i];
    }
    ref_rms_norm(x, nrm, d, N, m->rms_eps);
    mul_row_weight(nrm, (const float *) t[T_OUT_NORM], N, d);
    int lt;
    const void * lw = lm_head(m, t, &lt);
    ref_mul_mat(lt, lw, ref_row_size(lt, d), m->vocab, d, nrm, d, N, lg, m->vocab, threads);
    for (int i = 0; i < N; i++) {
        top1[i] = ref_argmax_first(lg + (size_t) i * m->vocab, m->vocab);
        if (logits) memcpy(logits + (size_t) i * m->vocab, lg + (size_t) i * m->vocab, sizeof(float) * m->vocab);
    }
    free(x);
    free(nrm);
    free(qkv);
    free(q);
    free(k);
    free(att);
    free(tmp);
    free(g);
    free(u);
    free(lg);
    free(mask);
}

/* ------------------------------------------------------------ Whisper -- */

/*
 * Whisper decoder step, batch 1 (models/whisper/ggml_decoder_graph.rs):
 * reusable one-token graph :3869-4052, self attention :4557-5044, cross
 * attention :5106-5340, MLP :5342-5392, LayerNorm :5953-6010, linear with
 * bias :5446-5490, cross K/V precompute :5780-5805.
 * Pointer table: per layer OA_WH_LAYER_KINDS (24) entries in the order of
 * oa_whisper_tensor_kind, then token embedding (Q8_0), position embedding
 * (f32), final LayerNorm weight and bias.
 */
typedef struct {
    int d_model, n_layers, n_head, ffn, vocab, max_positions, n_frames;
    float ln_eps;
    int ffn_act; /* FFN activation (nn/decoder.rs:1125-1138): 0 GELU, 1 RELU, 2 GELU_ERF, 3 SILU */
} ref_whisper_dims;

static float wh_act(int act, float x) {
    switch (act) {
        case 1: return ref_relu(x);
        case 2: return ref_gelu_erf(x);
        case 3: return ref_silu(x);
        default: return ref_gelu(x);
    }
}

enum {
    W_SELF_LN_W = 0, W_SELF_LN_B, W_SELF_Q, W_SELF_Q_B, W_SELF_K, W_SELF_V, W_SELF_V_B, W_SELF_O, W_SELF_O_B,
    W_CROSS_LN_W, W_CROSS_LN_B, W_CROSS_Q, W_CROSS_Q_B, W_CROSS_K, W_CROSS_V, W_CROSS_V_B, W_CROSS_O, W_CROSS_O_B,
    W_MLP_LN_W, W_MLP_LN_B, W_FC1, W_FC1_B, W_FC2, W_FC2_B, W_PER_LAYER
};

static const void * wp(const void * const * t, int layer, int kind) { return t[layer * W_PER_LAYER + kind]; }
static const void * wg(const ref_whisper_dims * m, const void * const * t, int i) {
    return t[m->n_layers * W_PER_LAYER + i];
}

/* apply_affine_layer_norm: norm, then * w, then + b (separate f32 ops) */
static void wh_layer_norm(const float * x, float * y, int n, const float * w, const float * b, float eps) {
    ref_norm(x, y, n, 1, eps);
    for (int i = 0; i < n; i++) y[i] = y[i] * w[i];
    for (int i = 0; i < n; i++) y[i] = y[i] + b[i];
}

/* mul_mat then + bias (when given) */
static void wh_linear(const void * w, int rows, int k, const float * x, const float * b, float * y, int threads) {
    ref_mul_mat(REF_Q8_0, w, ref_row_size(REF_Q8_0, k), rows, k, x, k, 1, y, rows, threads);
    if (b)
        for (int i = 0; i < rows; i++) y[i] = y[i] + b[i];
}

/* cross K/V for every layer: K = Wk enc, V = Wv enc + bv, f16 [n_frames][d] */
void ref_whisper_cross_kv(const ref_whisper_dims * m, const void * const * t, const float * enc,
                          uint16_t * const * ck, uint16_t * const * cv, int threads) {
    const int d = m->d_model, F = m->n_frames;
    float * k = (float *) malloc(sizeof(float) * (size_t) F * d);
    for (int l = 0; l < m->n_layers; l++) {
        ref_mul_mat(REF_Q8_0, wp(t, l, W_CROSS_K), ref_row_size(REF_Q8_0, d), d, d, enc, d, F, k, d, threads);
        ref_fp32_to_fp16_row(k, ck[l], (int64_t) F * d);
        ref_mul_mat(REF_Q8_0, wp(t, l, W_CROSS_V), ref_row_size(REF_Q8_0, d), d, d, enc, d, F, k, d, threads);
        const float * bv = (const float *) wp(t, l, W_CROSS_V_B);
        for (int f = 0; f < F; f++)
            for (int i = 0; i < d; i++) k[(size_t) f * d + i] = k[(size_t) f * d + i] + bv[i];
        ref_fp32_to_fp16_row(k, cv[l], (int64_t) F * d);
    }
    free(k);
}

/*
 * One token at position pos. kc/vc: per layer self K/V f16 [max_positions][d]
 * (row = position, all heads); ck/cv: per layer cross K/V f16 [n_frames][d].
 * Writes this position's K/V rows, attends over the full span with the
 * fixed-span mask (masked positions are skipped), fills logits [vocab] when
 * non-null and returns the first-max top-1.
 */
int32_t ref_whisper_step(const ref_whisper_dims * m, const void * const * t, uint16_t * const * kc,
                         uint16_t * const * vc, uint16_t * const * ck, uint16_t * const * cv, int32_t token, int pos,
                         float * logits, int fa_fidelity, int threads) {
    const int d = m->d_model, H = m->n_head, hd = d / H, mp = m->max_positions;
    float * x = (float *) malloc(sizeof(float) * d);
    float * nrm = (float *) malloc(sizeof(float) * d);
    float * q = (float *) malloc(sizeof(float) * d);
    float * k = (float *) malloc(sizeof(float) * d);
    float * v = (float *) malloc(sizeof(float) * d);
    float * att = (float *) malloc(sizeof(float) * d);
    float * o = (float *) malloc(sizeof(float) * d);
    float * h = (float *) malloc(sizeof(float) * m->ffn);
    uint16_t * mask = (uint16_t *) malloc(sizeof(uint16_t) * mp);
    for (int j = 0; j < mp; j++) mask[j] = j <= pos ? 0 : 0xFC00;
    /* token + learned position embedding */
    ref_dequantize_row_q8_0((const ref_block_q8_0 *) ((const char *) wg(m, t, 0) + (size_t) token * ref_row_size(REF_Q8_0, d)),
                            x, d);
    const float * pe = (const float *) wg(m, t, 1) + (size_t) pos * d;
    for (int i = 0; i < d; i++) x[i] = x[i] + pe[i];
    const float scale = 1.0f / sqrtf((float) hd);
    for (int l = 0; l < m->n_layers; l++) {
        /* self attention */
        wh_layer_norm(x, nrm, d, (const float *) wp(t, l, W_SELF_LN_W), (const float *) wp(t, l, W_SELF_LN_B), m->ln_eps);
        wh_linear(wp(t, l, W_SELF_Q), d, d, nrm, (const float *) wp(t, l, W_SELF_Q_B), q, threads);
        wh_linear(wp(t, l, W_SELF_K), d, d, nrm, NULL, k, threads);
        wh_linear(wp(t, l, W_SELF_V), d, d, nrm, (const float *) wp(t, l, W_SELF_V_B), v, threads);
        ref_fp32_to_fp16_row(k, kc[l] + (size_t) pos * d, d);
        ref_fp32_to_fp16_row(v, vc[l] + (size_t) pos * d, d);
        ref_flash_attn_ext(q, d, hd, kc[l], vc[l], hd, d, mask, mp, att, hd, 1, H, H, mp, scale, fa_fidelity, threads);
        wh_linear(wp(t, l, W_SELF_O), d, d, att, (const float *) wp(t, l, W_SELF_O_B), o, threads);
        for (int i = 0; i < d; i++) x[i] = o[i] + x[i];
        /* cross attention */
        wh_layer_norm(x, nrm, d, (const float *) wp(t, l, W_CROSS_LN_W), (const float *) wp(t, l, W_CROSS_LN_B), m->ln_eps);
        wh_linear(wp(t, l, W_CROSS_Q), d, d, nrm, (const float *) wp(t, l, W_CROSS_Q_B), q, threads);
        ref_flash_attn_ext(q, d, hd, ck[l], cv[l], hd, d, NULL, 0, att, hd, 1, H, H, m->n_frames, scale, fa_fidelity,
                           threads);
        wh_linear(wp(t, l, W_CROSS_O), d, d, att, (const float *) wp(t, l, W_CROSS_O_B), o, threads);
        for (int i = 0; i < d; i++) x[i] = o[i] + x[i];
        /* MLP */
        wh_layer_norm(x, nrm, d, (const float *) wp(t, l, W_MLP_LN_W), (const float *) wp(t, l, W_MLP_LN_B), m->ln_eps);
        wh_linear(wp(t, l, W_FC1), m->ffn, d, nrm, (const float *) wp(t, l, W_FC1_B), h, threads);
        for (int i = 0; i < m->ffn; i++) h[i] = wh_act(m->ffn_act, h[i]);
        wh_linear(wp(t, l, W_FC2), d, m->ffn, h, (const float *) wp(t, l, W_FC2_B), o, threads);
        for (int i = 0; i < d; i++) x[i] = o[i] + x[i];
    }
    wh_layer_norm(x, nrm, d, (const float *) wg(m, t, 2), (const float *) wg(m, t, 3), m->ln_eps);
    float * lg = logits ? logits : (float *) malloc(sizeof(float) * m->vocab);
    ref_mul_mat(REF_Q8_0, wg(m, t, 0), ref_row_size(REF_Q8_0, d), m->vocab, d, nrm, d, 1, lg, m->vocab, threads);
    const int32_t top1 = ref_argmax_first(lg, m->vocab);
    if (!logits) free(lg);
    free(x);
    free(nrm);
    free(q);
    free(k);
    free(v);
    free(att);
    free(o);
    free(h);
    free(mask);
    return top1;
}
