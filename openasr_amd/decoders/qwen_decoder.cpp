// qwen_decoder.cpp -- the Qwen3 LLM decoder as the OpenASR host drives it
// through ggml (declared in include/openasr_models.h).
//
// Graph construction follows the reference emitters op for op:
//   llm_layer                      crates/openasr-core/src/nn/decoder.rs:1850-2145
//   build_projected_qkv (fused)    nn/decoder.rs:1722-1789
//   compose_llm_decoder_layer_stack nn/decoder.rs:2206-2331
//   resident f16 KV arena, zeroed  nn/decoder.rs:2339-2422
//   fixed-span KV mask             nn/decoder.rs:2431-2463
//   reusable decode graph          models/qwen/llm_transformer.rs:5169-5320
//   fused logits + first-max top1  llm_transformer.rs:2096-2115
//   HIP-lane graph (a session option): expand_attention_kv
//   nn/decoder.rs:1799-1841 (native GQA Unsupported on HIP,
//   ggml_runtime/cpu_graph.rs:736-757), llm_naive_masked_attention
//   nn/decoder.rs:2154-2200 for prefill chunks of more than two queries over
//   a span of more than 32 positions (llm_transformer.rs:7864-7877), its
//   products at GGML_PREC_F32 (cpu_graph.rs:157-165, 202-228), even prefill
//   widths (llm_transformer.rs:3186-3198, 7903-7911)
// The batched logits head (one lm_head GEMV over every sequence, then a
// first-max argmax) replaces the reference's per-slot logits graphs
// (models/qwen/batched_decode.rs:961-975); its output is the same token.

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ggml_host.h"
#include "openasr_models.h"
#include "pack_reader.h"

using oa_pack::blob;
using oa_pack::pack_reader;

extern "C" void oa_synth_normal(uint64_t seed, uint64_t stream, int64_t first, int64_t n, float mean, float std_dev,
                                float * out);

namespace {

constexpr int kPrefillChunk = 256;  // llm_transformer.rs:60

struct qlayer_host {
    std::vector<float> attn_norm, q_norm, k_norm, ffn_norm;
    blob qkv, o, gate, up, down;
};

uint64_t stream_id(int layer, int kind, int part) { return (uint64_t) (layer + 1) * 1000 + (uint64_t) kind * 10 + part; }

// rows x k matrix N(0, 0.02) from one or more generator streams, quantized
std::vector<uint8_t> synth_matrix(int wtype, uint64_t seed, const std::vector<std::pair<uint64_t, int64_t>> & parts,
                                  int64_t k) {
    int64_t rows = 0;
    for (auto & p : parts) rows += p.second;
    const size_t rs = ggml_row_size((ggml_type) wtype, k);
    std::vector<uint8_t> out((size_t) rows * rs);
    // slabs of rows are independent (the generator is counter-based and the
    // quantizers work row by row), so they are filled in parallel
    const int64_t slab = 256;
    int64_t row0 = 0;
    for (auto & p : parts) {
        const int64_t n_slabs = (p.second + slab - 1) / slab;
#pragma omp parallel
        {
            std::vector<float> buf((size_t) (slab * k));  // one per thread, reused across slabs
#pragma omp for schedule(dynamic, 1)
            for (int64_t si = 0; si < n_slabs; si++) {
                const int64_t r = si * slab;
                const int64_t n = std::min(slab, p.second - r);
                oa_synth_normal(seed, p.first, r * k, n * k, 0.0f, 0.02f, buf.data());
                ggml_quantize_chunk((ggml_type) wtype, buf.data(), out.data() + (size_t) (row0 + r) * rs, 0, n, k,
                                    nullptr);
            }
        }
        row0 += p.second;
    }
    return out;
}

}  // namespace

struct oa_qwen_weights {
    oa_qwen_config cfg;
    blob tok_embd;
    blob lm_head;  // empty: the output projection is tied to tok_embd
    std::vector<float> out_norm;
    std::vector<qlayer_host> layers;
    oa_gguf * src = nullptr;  // the mapped pack the views point into
    ~oa_qwen_weights() { oa_gguf_close(src); }
};

struct qlayer_dev {
    ggml_tensor *attn_norm, *qkv, *q_norm, *k_norm, *o, *ffn_norm, *gate, *up, *down;
};

struct oa_qwen_model {
    oa_qwen_config cfg;
    ggml_backend_t backend;
    ggml_context * ctx;
    ggml_backend_buffer_t buf;
    ggml_tensor *tok_embd, *out_norm;
    ggml_tensor * lm_head;  // tok_embd when tied
    std::vector<qlayer_dev> layers;
};

struct step_graph {
    ggml_context * ctx = nullptr;
    ggml_cgraph * gf = nullptr;
    ggml_gallocr_t galloc = nullptr;
    ggml_tensor *tokens = nullptr, *hidden = nullptr, *rows = nullptr, *pos = nullptr, *mask = nullptr;
    ggml_tensor *top1 = nullptr, *logits = nullptr;
    int T = 0;
    void release() {
        if (galloc) ggml_gallocr_free(galloc);
        if (ctx) ggml_free(ctx);
        *this = step_graph();
    }
};

struct oa_qwen_session {
    oa_qwen_model * m;
    int n_seq;
    int max_pos;
    ggml_context * kv_ctx = nullptr;
    ggml_backend_buffer_t kv_buf = nullptr;
    std::vector<ggml_tensor *> k_cache, v_cache;
    std::vector<int> n_past;  // per sequence
    step_graph decode;
    std::vector<uint16_t> mask_host;
    // greedy top-1 through the reversed-row graph (cpu_graph.rs:3772-3810)
    // instead of ARGMAX_FIRST; rev_idx holds vocab - 1 .. 0
    bool reversed_top1 = false;
    ggml_tensor * rev_idx = nullptr;
    // the graph the host builds on a discrete-GPU HIP backend (one sequence):
    // K/V expanded to the query heads by REPEAT, the unfused attention chain
    // for wide prefill chunks, chunks of at most prefill_chunk positions
    // trimmed to even widths
    bool hip_lane = false;
    int prefill_chunk = kPrefillChunk;
    // the self-attention's flash-attention precision contract
    // (set_flash_attention_precision, llm_transformer.rs:3044-3053)
    int fa_prec = GGML_PREC_DEFAULT;
    // the quantized projections' MUL_MAT precision (GgmlMatmulPrecision,
    // cpu_graph.rs:142-146, 3624-3685): the decoder's projections take the
    // plain mul_mat (nn/decoder.rs:1621), i.e. the default
    int mm_prec = GGML_PREC_DEFAULT;
};

namespace {

const ggml_fp16_t kNegInf = 0xFC00;

// Greedy top-1 with first-max ties from ggml's ARGMAX, which keeps the last
// of equal maxima: every logits row is reversed by GET_ROWS (one element per
// row for a single column, the transposed matrix's rows otherwise), then
// ARGMAX; the caller maps a result r to vocab - 1 - r
// (cpu_graph.rs:3772-3810, llm_transformer.rs:2096-2115).
ggml_tensor * top1_reversed(ggml_context * ctx, ggml_tensor * logits, ggml_tensor * rev) {
    const int64_t V = logits->ne[0], n = logits->ne[1];
    ggml_tensor * r;
    if (n == 1) {
        r = ggml_get_rows(ctx, ggml_reshape_2d(ctx, logits, 1, V), rev);
        r = ggml_reshape_2d(ctx, ggml_cont(ctx, r), V, 1);
    } else {
        ggml_tensor * tr = ggml_cont(ctx, ggml_transpose(ctx, logits));  // [n, V]
        r = ggml_cont(ctx, ggml_transpose(ctx, ggml_get_rows(ctx, tr, rev)));
    }
    return ggml_argmax(ctx, r);
}

ggml_tensor * rms_norm_mul(ggml_context * ctx, ggml_tensor * x, ggml_tensor * w, float eps) {
    return ggml_mul(ctx, ggml_rms_norm(ctx, x, eps), w);  // nn/norm.rs:39-56
}

// a quantized projection at the session's MUL_MAT precision
ggml_tensor * proj(ggml_context * ctx, ggml_tensor * w, ggml_tensor * x, int mm_prec) {
    ggml_tensor * y = ggml_mul_mat(ctx, w, x);
    if (mm_prec == GGML_PREC_F32) ggml_mul_mat_set_prec(y, GGML_PREC_F32);
    return y;
}

// llm_layer for token_count tokens of n_seq sequences (nn/decoder.rs:1850-2145)
ggml_tensor * llm_layer(ggml_context * ctx, const oa_qwen_config & c, const qlayer_dev & L, ggml_tensor * hidden,
                        ggml_tensor * k_hist, ggml_tensor * v_hist, ggml_tensor * rows, ggml_tensor * pos,
                        ggml_tensor * mask, int T, int n_seq, int max_pos, bool hip_lane, int fa_prec,
                        int mm_prec) {
    const int hd = c.head_dim, q_w = c.n_head * hd, kv_w = c.n_kv_head * hd;
    const int tokens = T * n_seq;
    ggml_tensor * normed = rms_norm_mul(ctx, hidden, L.attn_norm, c.rms_eps);
    // fused [q|k|v] projection then f32 column views (nn/decoder.rs:1722-1789)
    ggml_tensor * qkv = proj(ctx, L.qkv, normed, mm_prec);
    const size_t col = (size_t) (q_w + 2 * kv_w) * sizeof(float);
    ggml_tensor * q = ggml_view_2d(ctx, qkv, q_w, tokens, col, 0);
    ggml_tensor * k = ggml_view_2d(ctx, qkv, kv_w, tokens, col, (size_t) q_w * sizeof(float));
    ggml_tensor * v = ggml_view_2d(ctx, qkv, kv_w, tokens, col, (size_t) (q_w + kv_w) * sizeof(float));
    if (tokens > 1) {
        q = ggml_cont(ctx, q);
        k = ggml_cont(ctx, k);
        v = ggml_cont(ctx, v);
    }
    q = ggml_reshape_3d(ctx, q, hd, c.n_head, tokens);
    k = ggml_reshape_3d(ctx, k, hd, c.n_kv_head, tokens);
    v = ggml_reshape_3d(ctx, v, hd, c.n_kv_head, tokens);
    q = rms_norm_mul(ctx, q, L.q_norm, c.rms_eps);  // QK-norm per head (nn/decoder.rs:1937-1958)
    k = rms_norm_mul(ctx, k, L.k_norm, c.rms_eps);
    // RoPE NEOX, theta from the config, no YaRN (cpu_graph.rs:1135-1161)
    q = ggml_rope_ext(ctx, q, pos, nullptr, hd, GGML_ROPE_TYPE_NEOX, max_pos, c.rope_theta, 1.0f, 0.0f, 1.0f, 32.0f,
                      1.0f);
    k = ggml_rope_ext(ctx, k, pos, nullptr, hd, GGML_ROPE_TYPE_NEOX, max_pos, c.rope_theta, 1.0f, 0.0f, 1.0f, 32.0f,
                      1.0f);
    ggml_tensor *q_fa, *k_new, *v_new;
    if (T == 1) {
        // decode: [hd, heads, n_seq] -> [hd, 1, heads, n_seq] (nn/decoder.rs:1970-2000)
        if (n_seq == 1) {
            q_fa = ggml_permute(ctx, q, 0, 2, 1, 3);
            k_new = ggml_permute(ctx, k, 0, 2, 1, 3);
            v_new = ggml_permute(ctx, v, 0, 2, 1, 3);
        } else {
            q_fa = ggml_permute(ctx, q, 0, 2, 3, 1);
            k_new = ggml_permute(ctx, k, 0, 2, 3, 1);
            v_new = ggml_permute(ctx, v, 0, 2, 3, 1);
        }
    } else {
        q_fa = ggml_permute(ctx, ggml_reshape_4d(ctx, q, hd, c.n_head, T, n_seq), 0, 2, 1, 3);
        k_new = ggml_permute(ctx, ggml_reshape_4d(ctx, k, hd, c.n_kv_head, T, n_seq), 0, 2, 1, 3);
        v_new = ggml_permute(ctx, ggml_reshape_4d(ctx, v, hd, c.n_kv_head, T, n_seq), 0, 2, 1, 3);
    }
    // write this step's K/V into the resident cache, attend over the full span
    ggml_tensor * k_full = ggml_set_rows(ctx, k_hist, k_new, rows);
    ggml_tensor * v_full = ggml_set_rows(ctx, v_hist, v_new, rows);
    const int g = c.n_head / c.n_kv_head;
    if (hip_lane && n_seq == 1 && g > 1) {
        // expand_attention_kv: each kv head repeated for its query heads
        k_full = ggml_reshape_4d(ctx, k_full, hd, max_pos, 1, c.n_kv_head);
        v_full = ggml_reshape_4d(ctx, v_full, hd, max_pos, 1, c.n_kv_head);
        k_full = ggml_repeat_4d(ctx, k_full, hd, max_pos, g, c.n_kv_head);
        v_full = ggml_repeat_4d(ctx, v_full, hd, max_pos, g, c.n_kv_head);
        k_full = ggml_reshape_3d(ctx, k_full, hd, max_pos, c.n_head);
        v_full = ggml_reshape_3d(ctx, v_full, hd, max_pos, c.n_head);
    }
    const float scale = 1.0f / std::sqrt((float) hd);
    ggml_tensor * att;
    if (hip_lane && T > 2 && max_pos > 32) {
        // llm_naive_masked_attention: scores, masked softmax, V^T, context
        ggml_tensor * scores = ggml_mul_mat(ctx, k_full, q_fa);
        ggml_mul_mat_set_prec(scores, GGML_PREC_F32);
        ggml_tensor * probs = ggml_soft_max_ext(ctx, scores, mask, scale, 0.0f);
        ggml_tensor * v_t = ggml_cont(ctx, ggml_transpose(ctx, v_full));
        ggml_tensor * ctx_rows = ggml_mul_mat(ctx, v_t, probs);
        ggml_mul_mat_set_prec(ctx_rows, GGML_PREC_F32);
        att = ggml_cont(ctx, ggml_permute(ctx, ctx_rows, 0, 2, 1, 3));
    } else {
        att = ggml_flash_attn_ext(ctx, q_fa, k_full, v_full, mask, scale, 0.0f, 0.0f);
        ggml_flash_attn_ext_set_prec(att, (ggml_prec) fa_prec);
    }
    att = ggml_reshape_2d(ctx, att, q_w, tokens);
    ggml_tensor * post_attn = ggml_add(ctx, hidden, proj(ctx, L.o, att, mm_prec));
    // SwiGLU FFN with residual (nn/ffn.rs:64-91)
    ggml_tensor * ffn_in = rms_norm_mul(ctx, post_attn, L.ffn_norm, c.rms_eps);
    ggml_tensor * gate = ggml_silu(ctx, proj(ctx, L.gate, ffn_in, mm_prec));
    ggml_tensor * up = proj(ctx, L.up, ffn_in, mm_prec);
    ggml_tensor * down = proj(ctx, L.down, ggml_mul(ctx, gate, up), mm_prec);
    return ggml_add(ctx, down, post_attn);
}

size_t graph_ctx_bytes(int n_layers) {
    const size_t n_tensors = (size_t) n_layers * 64 + 256;
    return ggml_tensor_overhead() * n_tensors + ggml_graph_overhead_custom(n_tensors, false) + (1u << 16);
}

// one step graph: T positions of each sequence; hidden input when emb, else token ids
bool build_step(oa_qwen_session * s, step_graph & g, int T, bool emb) {
    const oa_qwen_model * m = s->m;
    const oa_qwen_config & c = m->cfg;
    const int n_seq = s->n_seq;
    ggml_init_params ip = {graph_ctx_bytes(c.n_layers), nullptr, true};
    g.ctx = ggml_init(ip);
    if (!g.ctx) return false;
    g.T = T;
    ggml_tensor * state;
    if (emb) {
        g.hidden = ggml_new_tensor_2d(g.ctx, GGML_TYPE_F32, c.d_model, (int64_t) T * n_seq);
        ggml_set_input(g.hidden);
        state = g.hidden;
    } else {
        g.tokens = ggml_new_tensor_1d(g.ctx, GGML_TYPE_I32, (int64_t) T * n_seq);
        ggml_set_input(g.tokens);
        state = ggml_get_rows(g.ctx, m->tok_embd, g.tokens);
    }
    g.rows = ggml_new_tensor_4d(g.ctx, GGML_TYPE_I32, T, 1, n_seq, 1);
    g.pos = ggml_new_tensor_1d(g.ctx, GGML_TYPE_I32, (int64_t) T * n_seq);
    g.mask = ggml_new_tensor_4d(g.ctx, GGML_TYPE_F16, s->max_pos, T, 1, n_seq);
    ggml_set_input(g.rows);
    ggml_set_input(g.pos);
    ggml_set_input(g.mask);
    for (int l = 0; l < c.n_layers; l++) {
        state = llm_layer(g.ctx, c, m->layers[(size_t) l], state, s->k_cache[(size_t) l], s->v_cache[(size_t) l],
                          g.rows, g.pos, g.mask, T, n_seq, s->max_pos, s->hip_lane, s->fa_prec, s->mm_prec);
    }
    ggml_tensor * last = state;
    if (T > 1) {  // the last position of each sequence
        last = ggml_cont(g.ctx, ggml_view_2d(g.ctx, state, c.d_model, n_seq, (size_t) T * c.d_model * sizeof(float),
                                             (size_t) (T - 1) * c.d_model * sizeof(float)));
    }
    ggml_tensor * normed = rms_norm_mul(g.ctx, last, m->out_norm, c.rms_eps);
    g.logits = proj(g.ctx, m->lm_head, normed, s->mm_prec);
    g.top1 = s->reversed_top1 ? top1_reversed(g.ctx, g.logits, s->rev_idx) : ggml_argmax_first(g.ctx, g.logits);
    ggml_set_output(g.logits);
    ggml_set_output(g.top1);
    g.gf = ggml_new_graph_custom(g.ctx, (size_t) c.n_layers * 64 + 256, false);
    ggml_build_forward_expand(g.gf, g.top1);
    g.galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m->backend));
    return ggml_gallocr_alloc_graph(g.galloc, g.gf);
}

// upload per-step inputs for positions [p0_s, p0_s + T) of every sequence
void set_step_inputs(oa_qwen_session * s, step_graph & g, int T) {
    const int n_seq = s->n_seq, mp = s->max_pos;
    std::vector<int32_t> rows((size_t) T * n_seq), pos((size_t) T * n_seq);
    std::vector<ggml_fp16_t> mask((size_t) mp * T * n_seq, kNegInf);
    for (int q = 0; q < n_seq; q++) {
        for (int t = 0; t < T; t++) {
            const int p = s->n_past[(size_t) q] + t;
            rows[(size_t) q * T + t] = p;
            pos[(size_t) q * T + t] = p;
            ggml_fp16_t * mr = mask.data() + ((size_t) q * T + t) * mp;
            for (int j = 0; j <= p; j++) mr[j] = 0;  // fixed-span mask (nn/decoder.rs:2431-2463)
        }
    }
    ggml_backend_tensor_set(g.rows, rows.data(), 0, rows.size() * 4);
    ggml_backend_tensor_set(g.pos, pos.data(), 0, pos.size() * 4);
    ggml_backend_tensor_set(g.mask, mask.data(), 0, mask.size() * 2);
}

// the step's greedy tokens; a reversed-row result r is vocab - 1 - r, and a
// value outside the vocabulary fails the step (llm_transformer.rs:2117-2130)
int read_top1(const oa_qwen_session * s, const step_graph & g, int32_t * out) {
    ggml_backend_tensor_get(g.top1, out, 0, (size_t) s->n_seq * sizeof(int32_t));
    if (!s->reversed_top1) return GGML_STATUS_SUCCESS;
    const int V = s->m->cfg.vocab;
    for (int q = 0; q < s->n_seq; q++) {
        if (out[q] < 0 || out[q] >= V) return GGML_STATUS_FAILED;
        out[q] = V - 1 - out[q];
    }
    return GGML_STATUS_SUCCESS;
}

int run_chunk(oa_qwen_session * s, const void * input, bool emb, int T, int32_t * top1_out) {
    step_graph g;
    if (!build_step(s, g, T, emb)) {
        g.release();
        return GGML_STATUS_ALLOC_FAILED;
    }
    const oa_qwen_config & c = s->m->cfg;
    if (emb) ggml_backend_tensor_set(g.hidden, input, 0, (size_t) T * s->n_seq * c.d_model * sizeof(float));
    else ggml_backend_tensor_set(g.tokens, input, 0, (size_t) T * s->n_seq * sizeof(int32_t));
    set_step_inputs(s, g, T);
    const int st = ggml_backend_graph_compute(s->m->backend, g.gf);
    int ret = st;
    if (st == GGML_STATUS_SUCCESS) {
        for (int q = 0; q < s->n_seq; q++) s->n_past[(size_t) q] += T;
        if (top1_out) ret = read_top1(s, g, top1_out);
    }
    g.release();
    return ret;
}

}  // namespace

extern "C" {

oa_qwen_weights * oa_qwen_weights_synthesize(const oa_qwen_config * cfg) {
    oa_qwen_weights * w = new oa_qwen_weights;
    w->cfg = *cfg;
    const oa_qwen_config & c = *cfg;
    const int q_w = c.n_head * c.head_dim, kv_w = c.n_kv_head * c.head_dim;
    w->tok_embd = synth_matrix(c.wtype, c.seed, {{stream_id(-1, OA_QWEN_TOKEN_EMBD, 0), c.vocab}}, c.d_model);
    w->out_norm.assign((size_t) c.d_model, 1.0f);
    w->layers.resize((size_t) c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        qlayer_host & L = w->layers[(size_t) l];
        L.attn_norm.assign((size_t) c.d_model, 1.0f);
        L.ffn_norm.assign((size_t) c.d_model, 1.0f);
        L.q_norm.assign((size_t) c.head_dim, 1.0f);
        L.k_norm.assign((size_t) c.head_dim, 1.0f);
        // q, k and v drawn separately, then row-concatenated as the fused weight
        // (llm_transformer.rs:6505-6555)
        L.qkv = synth_matrix(c.wtype, c.seed,
                             {{stream_id(l, OA_QWEN_QKV, 0), q_w}, {stream_id(l, OA_QWEN_QKV, 1), kv_w},
                              {stream_id(l, OA_QWEN_QKV, 2), kv_w}},
                             c.d_model);
        L.o = synth_matrix(c.wtype, c.seed, {{stream_id(l, OA_QWEN_O, 0), c.d_model}}, q_w);
        L.gate = synth_matrix(c.wtype, c.seed, {{stream_id(l, OA_QWEN_GATE, 0), c.ffn}}, c.d_model);
        L.up = synth_matrix(c.wtype, c.seed, {{stream_id(l, OA_QWEN_UP, 0), c.ffn}}, c.d_model);
        L.down = synth_matrix(c.wtype, c.seed, {{stream_id(l, OA_QWEN_DOWN, 0), c.d_model}}, c.ffn);
    }
    return w;
}

void oa_qwen_weights_free(oa_qwen_weights * w) { delete w; }

const void * oa_qwen_weights_tensor(const oa_qwen_weights * w, int layer, int kind, size_t * nbytes) {
    auto ret_u8 = [&](const blob & v) -> const void * {
        if (nbytes) *nbytes = v.size();
        return v.data();
    };
    auto ret_f = [&](const std::vector<float> & v) -> const void * {
        if (nbytes) *nbytes = v.size() * sizeof(float);
        return v.data();
    };
    if (kind == OA_QWEN_TOKEN_EMBD) return ret_u8(w->tok_embd);
    if (kind == OA_QWEN_OUTPUT) return w->lm_head.size() ? ret_u8(w->lm_head) : nullptr;
    if (kind == OA_QWEN_OUTPUT_NORM) return ret_f(w->out_norm);
    if (layer < 0 || layer >= (int) w->layers.size()) return nullptr;
    const qlayer_host & L = w->layers[(size_t) layer];
    switch (kind) {
        case OA_QWEN_ATTN_NORM: return ret_f(L.attn_norm);
        case OA_QWEN_QKV: return ret_u8(L.qkv);
        case OA_QWEN_Q_NORM: return ret_f(L.q_norm);
        case OA_QWEN_K_NORM: return ret_f(L.k_norm);
        case OA_QWEN_O: return ret_u8(L.o);
        case OA_QWEN_FFN_NORM: return ret_f(L.ffn_norm);
        case OA_QWEN_GATE: return ret_u8(L.gate);
        case OA_QWEN_UP: return ret_u8(L.up);
        case OA_QWEN_DOWN: return ret_u8(L.down);
        default: return nullptr;
    }
}

oa_qwen_model * oa_qwen_model_create(ggml_backend_t backend, const oa_qwen_weights * w) {
    const oa_qwen_config & c = w->cfg;
    oa_qwen_model * m = new oa_qwen_model;
    m->cfg = c;
    m->backend = backend;
    ggml_init_params ip = {ggml_tensor_overhead() * ((size_t) c.n_layers * 12 + 16), nullptr, true};
    m->ctx = ggml_init(ip);
    const ggml_type wt = (ggml_type) c.wtype;
    const int q_w = c.n_head * c.head_dim, kv_w = c.n_kv_head * c.head_dim;
    m->tok_embd = ggml_new_tensor_2d(m->ctx, wt, c.d_model, c.vocab);
    m->lm_head = w->lm_head.size() ? ggml_new_tensor_2d(m->ctx, (ggml_type) c.out_wtype, c.d_model, c.vocab)
                                   : m->tok_embd;
    m->out_norm = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, c.d_model);
    m->layers.resize((size_t) c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        qlayer_dev & L = m->layers[(size_t) l];
        L.attn_norm = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, c.d_model);
        L.qkv = ggml_new_tensor_2d(m->ctx, wt, c.d_model, q_w + 2 * kv_w);
        L.q_norm = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, c.head_dim);
        L.k_norm = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, c.head_dim);
        L.o = ggml_new_tensor_2d(m->ctx, wt, q_w, c.d_model);
        L.ffn_norm = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, c.d_model);
        L.gate = ggml_new_tensor_2d(m->ctx, wt, c.d_model, c.ffn);
        L.up = ggml_new_tensor_2d(m->ctx, wt, c.d_model, c.ffn);
        L.down = ggml_new_tensor_2d(m->ctx, wt, c.ffn, c.d_model);
    }
    m->buf = ggml_backend_alloc_ctx_tensors_from_buft(m->ctx, ggml_backend_get_default_buffer_type(backend));
    if (!m->buf) {
        ggml_free(m->ctx);
        delete m;
        return nullptr;
    }
    ggml_backend_buffer_set_usage(m->buf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    auto up = [](ggml_tensor * t, const void * data, size_t n) { ggml_backend_tensor_set(t, data, 0, n); };
    up(m->tok_embd, w->tok_embd.data(), w->tok_embd.size());
    if (m->lm_head != m->tok_embd) up(m->lm_head, w->lm_head.data(), w->lm_head.size());
    up(m->out_norm, w->out_norm.data(), w->out_norm.size() * 4);
    for (int l = 0; l < c.n_layers; l++) {
        const qlayer_host & H = w->layers[(size_t) l];
        qlayer_dev & L = m->layers[(size_t) l];
        up(L.attn_norm, H.attn_norm.data(), H.attn_norm.size() * 4);
        up(L.qkv, H.qkv.data(), H.qkv.size());
        up(L.q_norm, H.q_norm.data(), H.q_norm.size() * 4);
        up(L.k_norm, H.k_norm.data(), H.k_norm.size() * 4);
        up(L.o, H.o.data(), H.o.size());
        up(L.ffn_norm, H.ffn_norm.data(), H.ffn_norm.size() * 4);
        up(L.gate, H.gate.data(), H.gate.size());
        up(L.up, H.up.data(), H.up.size());
        up(L.down, H.down.data(), H.down.size());
    }
    return m;
}

void oa_qwen_model_free(oa_qwen_model * m) {
    if (!m) return;
    ggml_backend_buffer_free(m->buf);
    ggml_free(m->ctx);
    delete m;
}

oa_qwen_session * oa_qwen_session_create(oa_qwen_model * m, int n_seq, int max_positions) {
    const oa_qwen_config & c = m->cfg;
    oa_qwen_session * s = new oa_qwen_session;
    s->m = m;
    s->n_seq = n_seq;
    s->max_pos = max_positions;
    s->n_past.assign((size_t) n_seq, 0);
    ggml_init_params ip = {ggml_tensor_overhead() * ((size_t) c.n_layers * 2 + 4), nullptr, true};
    s->kv_ctx = ggml_init(ip);
    for (int l = 0; l < c.n_layers; l++) {
        s->k_cache.push_back(ggml_new_tensor_4d(s->kv_ctx, GGML_TYPE_F16, c.head_dim, max_positions, c.n_kv_head, n_seq));
        s->v_cache.push_back(ggml_new_tensor_4d(s->kv_ctx, GGML_TYPE_F16, c.head_dim, max_positions, c.n_kv_head, n_seq));
    }
    s->rev_idx = ggml_new_tensor_1d(s->kv_ctx, GGML_TYPE_I32, c.vocab);
    s->kv_buf = ggml_backend_alloc_ctx_tensors_from_buft(s->kv_ctx, ggml_backend_get_default_buffer_type(m->backend));
    if (!s->kv_buf) {
        ggml_free(s->kv_ctx);
        delete s;
        return nullptr;
    }
    ggml_backend_buffer_clear(s->kv_buf, 0);  // unwritten slots stay zero (nn/decoder.rs:2407-2416)
    std::vector<int32_t> rev((size_t) c.vocab);
    for (int i = 0; i < c.vocab; i++) rev[(size_t) i] = c.vocab - 1 - i;
    ggml_backend_tensor_set(s->rev_idx, rev.data(), 0, rev.size() * sizeof(int32_t));
    return s;
}

void oa_qwen_session_free(oa_qwen_session * s) {
    if (!s) return;
    s->decode.release();
    ggml_backend_buffer_free(s->kv_buf);
    ggml_free(s->kv_ctx);
    delete s;
}

int oa_qwen_session_position(const oa_qwen_session * s, int seq) { return s->n_past[(size_t) seq]; }

int oa_qwen_session_set_hip_lane(oa_qwen_session * s, int enable, int prefill_chunk) {
    // the host refuses more than one sequence on this lane
    // (llm_transformer.rs:2444-2450)
    if (enable && (s->n_seq != 1 || prefill_chunk < 1)) return GGML_STATUS_FAILED;
    s->hip_lane = enable != 0;
    s->prefill_chunk = enable ? prefill_chunk : kPrefillChunk;
    s->decode.release();  // rebuilt with the lane's graph on the next step
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_session_set_flash_attention_precision(oa_qwen_session * s, int precision) {
    if (precision != GGML_PREC_DEFAULT && precision != GGML_PREC_F32) return GGML_STATUS_FAILED;
    s->fa_prec = precision;
    s->decode.release();  // no graph built under the other contract survives
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_session_set_matmul_precision(oa_qwen_session * s, int precision) {
    if (precision != GGML_PREC_DEFAULT && precision != GGML_PREC_F32) return GGML_STATUS_FAILED;
    s->mm_prec = precision;
    s->decode.release();  // no graph built under the other contract survives
    return GGML_STATUS_SUCCESS;
}

void oa_qwen_session_set_reversed_top1(oa_qwen_session * s, int enable) {
    if (s->reversed_top1 == (enable != 0)) return;
    s->reversed_top1 = enable != 0;
    s->decode.release();  // rebuilt with the other head on the next step
}

// width of the next prefill chunk: at most the session's chunk; on the HIP
// lane an odd width above one is trimmed by one, so every multi-token chunk
// is even and a final single token follows (even_prefill_chunk_len,
// llm_transformer.rs:7903-7911)
static int chunk_width(const oa_qwen_session * s, int remaining) {
    const int w = std::min(s->hip_lane ? s->prefill_chunk : kPrefillChunk, remaining);
    return s->hip_lane && w > 1 && w % 2 == 1 ? w - 1 : w;
}

int oa_qwen_prefill_embeddings(oa_qwen_session * s, const float * emb, int T, int32_t * top1_out) {
    const int d = s->m->cfg.d_model, n_seq = s->n_seq;
    for (int t0 = 0, n = 0; t0 < T; t0 += n) {
        n = chunk_width(s, T - t0);
        std::vector<float> chunk((size_t) n * n_seq * d);
        for (int q = 0; q < n_seq; q++) {
            std::memcpy(chunk.data() + (size_t) q * n * d, emb + ((size_t) q * T + t0) * d, (size_t) n * d * 4);
        }
        const int st = run_chunk(s, chunk.data(), true, n, t0 + n == T ? top1_out : nullptr);
        if (st != GGML_STATUS_SUCCESS) return st;
    }
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_prefill_tokens(oa_qwen_session * s, const int32_t * tokens, int T, int32_t * top1_out) {
    const int n_seq = s->n_seq;
    for (int t0 = 0, n = 0; t0 < T; t0 += n) {
        n = chunk_width(s, T - t0);
        std::vector<int32_t> chunk((size_t) n * n_seq);
        for (int q = 0; q < n_seq; q++) {
            std::memcpy(chunk.data() + (size_t) q * n, tokens + (size_t) q * T + t0, (size_t) n * 4);
        }
        const int st = run_chunk(s, chunk.data(), false, n, t0 + n == T ? top1_out : nullptr);
        if (st != GGML_STATUS_SUCCESS) return st;
    }
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_decode_step(oa_qwen_session * s, const int32_t * tokens, int32_t * top1_out, float * logits_out) {
    if (!s->decode.gf && !build_step(s, s->decode, 1, false)) {
        s->decode.release();
        return GGML_STATUS_ALLOC_FAILED;
    }
    for (int q = 0; q < s->n_seq; q++) {
        if (s->n_past[(size_t) q] >= s->max_pos) return GGML_STATUS_FAILED;
    }
    step_graph & g = s->decode;
    ggml_backend_tensor_set(g.tokens, tokens, 0, (size_t) s->n_seq * 4);
    set_step_inputs(s, g, 1);
    const int st = ggml_backend_graph_compute(s->m->backend, g.gf);
    if (st != GGML_STATUS_SUCCESS) return st;
    for (int q = 0; q < s->n_seq; q++) s->n_past[(size_t) q] += 1;
    if (top1_out) {
        const int rt = read_top1(s, g, top1_out);
        if (rt != GGML_STATUS_SUCCESS) return rt;
    }
    if (logits_out) ggml_backend_tensor_get(g.logits, logits_out, 0, (size_t) s->n_seq * s->m->cfg.vocab * 4);
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_generate(oa_qwen_session * s, const int32_t * first_tokens, int n_steps, int32_t * out_tokens,
                     double * step_ms) {
    std::vector<int32_t> cur(first_tokens, first_tokens + s->n_seq);
    for (int i = 0; i < n_steps; i++) {
        const auto t0 = std::chrono::steady_clock::now();
        const int st = oa_qwen_decode_step(s, cur.data(), out_tokens + (size_t) i * s->n_seq, nullptr);
        if (step_ms) step_ms[i] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        if (st != GGML_STATUS_SUCCESS) return st;
        std::memcpy(cur.data(), out_tokens + (size_t) i * s->n_seq, (size_t) s->n_seq * 4);
    }
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_read_kv(const oa_qwen_session * s, int layer, int seq, uint16_t * k_out, uint16_t * v_out) {
    const oa_qwen_config & c = s->m->cfg;
    const size_t plane = (size_t) c.head_dim * s->max_pos * c.n_kv_head * 2;
    if (k_out && ggml_backend_tensor_get(s->k_cache[(size_t) layer], k_out, plane * seq, plane)) return 1;
    if (v_out && ggml_backend_tensor_get(s->v_cache[(size_t) layer], v_out, plane * seq, plane)) return 1;
    return 0;
}

struct ggml_cgraph * oa_qwen_decode_graph(oa_qwen_session * s) { return s->decode.gf; }

int oa_detect_degenerate_ngram(const int32_t * tokens, int len, int max_ngram, const int * bounds, int * ngram_len,
                               int * repeats) {
    if (!tokens || len <= 0) return -1;
    for (int n = 1; n <= max_ngram; n++) {
        // the bound for this cycle length: the caller's, else the shipped
        // tiers (seq2seq_greedy_decode.rs:51-58); 0 disables this length
        const int bound = bounds ? bounds[n - 1] : (n == 1 ? 8 : (n == 2 ? 6 : 4));
        if (bound <= 0) continue;
        if ((int64_t) len < (int64_t) n * bound) continue;
        const int32_t * tail = tokens + len - n;
        int r = 1;
        while ((int64_t) (r + 1) * n <= len && std::memcmp(tokens + len - (r + 1) * n, tail, (size_t) n * 4) == 0) r++;
        if (r >= bound) {
            if (ngram_len) *ngram_len = n;
            if (repeats) *repeats = r;
            return len - (r - 1) * n;
        }
    }
    return -1;
}

}  // extern "C"

// ------------------------------------------------------- runtime packs ----

extern "C" oa_qwen_weights * oa_qwen_weights_load_gguf(const char * path, char * err, size_t err_cap) {
    auto report = [&](const std::string & msg) -> oa_qwen_weights * {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", msg.c_str());
        return nullptr;
    };
    char gerr[256] = {0};
    oa_gguf * g = oa_gguf_open(path, gerr, sizeof(gerr));
    if (!g) return report(gerr);
    oa_qwen_weights * w = new oa_qwen_weights;
    w->src = g;
    pack_reader r{g, {}};
    auto bad = [&](const std::string & msg) {
        delete w;
        return report(msg);
    };
    // OpenASR package metadata (oasr_metadata.rs:15-28): present keys must be valid
    if (const char * v = oa_gguf_get_str(g, "openasr.package.version"); v && std::strcmp(v, "1") != 0)
        return bad(std::string("unsupported openasr.package.version ") + v);
    if (oa_gguf_kv_type(g, "openasr.package.version") >= 0 && !oa_gguf_get_str(g, "openasr.package.version"))
        return bad("openasr.package.version is not a string");
    if (const char * a = oa_gguf_get_str(g, "general.architecture"); a && std::strcmp(a, "qwen3-asr") != 0)
        return bad(std::string("general.architecture is ") + a + ", not qwen3-asr");
    oa_qwen_config & c = w->cfg;
    c = oa_qwen_config{};
    if (!r.key_i("qwen3-asr.llm.n_layers", c.n_layers) || !r.key_i("qwen3-asr.llm.d_model", c.d_model) ||
        !r.key_i("qwen3-asr.llm.n_heads", c.n_head) || !r.key_i("qwen3-asr.llm.n_kv_heads", c.n_kv_head) ||
        !r.key_i("qwen3-asr.llm.head_dim", c.head_dim) || !r.key_i("qwen3-asr.llm.vocab_size", c.vocab))
        return bad(r.err);
    if (c.n_head % c.n_kv_head != 0) return bad("n_heads is not a multiple of n_kv_heads");
    double theta = 1e6;
    if (oa_gguf_kv_type(g, "qwen3-asr.llm.rope_theta") >= 0 && !oa_gguf_get_f64(g, "qwen3-asr.llm.rope_theta", &theta))
        return bad("qwen3-asr.llm.rope_theta is not a number");
    c.rope_theta = (float) theta;
    c.rms_eps = 1e-6f;
    // matrix type and FFN width from the first layer's gate projection
    const int64_t gi = oa_gguf_find_tensor(g, "blk.0.ffn_gate.weight");
    if (gi < 0) return bad("missing tensor blk.0.ffn_gate.weight");
    int64_t ne[4];
    oa_gguf_tensor_info(g, gi, &c.wtype, ne);
    if (c.wtype != GGML_TYPE_Q8_0 && c.wtype != GGML_TYPE_Q4_K)
        return bad(std::string("matrices are ") + ggml_type_name((ggml_type) c.wtype) + ", not Q8_0 or Q4_K");
    c.ffn = (int) ne[1];
    const int q_w = c.n_head * c.head_dim, kv_w = c.n_kv_head * c.head_dim;
    if (!r.mat("token_embd.weight", c.d_model, c.vocab, c.wtype, w->tok_embd) ||
        !r.vec("output_norm.weight", c.d_model, w->out_norm))
        return bad(r.err);
    if (oa_gguf_find_tensor(g, "output.weight") >= 0) {
        int ot = 0;
        const int64_t oi = r.tensor("output.weight", c.d_model, c.vocab, {GGML_TYPE_Q8_0, GGML_TYPE_Q4_K}, ot);
        if (oi < 0) return bad(r.err);
        size_t nb = 0;
        const void * p = oa_gguf_tensor_data(g, oi, &nb);
        // byte-identical to the embedding: tied after all
        if (ot != c.wtype || nb != w->tok_embd.size() || std::memcmp(p, w->tok_embd.data(), nb) != 0) {
            w->lm_head.set_view(p, nb);
            c.out_wtype = ot;
        }
    }
    w->layers.resize((size_t) c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        qlayer_host & L = w->layers[(size_t) l];
        const std::string p = "blk." + std::to_string(l) + ".";
        blob q, k, v;
        if (!r.vec(p + "attn_norm.weight", c.d_model, L.attn_norm) ||
            !r.vec(p + "attn_q_norm.weight", c.head_dim, L.q_norm) ||
            !r.vec(p + "attn_k_norm.weight", c.head_dim, L.k_norm) ||
            !r.vec(p + "ffn_norm.weight", c.d_model, L.ffn_norm) ||
            !r.mat(p + "attn_q.weight", c.d_model, q_w, c.wtype, q) ||
            !r.mat(p + "attn_k.weight", c.d_model, kv_w, c.wtype, k) ||
            !r.mat(p + "attn_v.weight", c.d_model, kv_w, c.wtype, v) ||
            !r.mat(p + "attn_output.weight", q_w, c.d_model, c.wtype, L.o) ||
            !r.mat(p + "ffn_gate.weight", c.d_model, c.ffn, c.wtype, L.gate) ||
            !r.mat(p + "ffn_up.weight", c.d_model, c.ffn, c.wtype, L.up) ||
            !r.mat(p + "ffn_down.weight", c.ffn, c.d_model, c.wtype, L.down))
            return bad(r.err);
        // the fused projection: rows of q, then k, then v (llm_transformer.rs:6505-6555)
        std::vector<uint8_t> qkv(q.size() + k.size() + v.size());
        std::memcpy(qkv.data(), q.data(), q.size());
        std::memcpy(qkv.data() + q.size(), k.data(), k.size());
        std::memcpy(qkv.data() + q.size() + k.size(), v.data(), v.size());
        L.qkv = std::move(qkv);
    }
    return w;
}

extern "C" void oa_qwen_weights_config(const oa_qwen_weights * w, oa_qwen_config * out) { *out = w->cfg; }
