// whisper_decoder.cpp -- the Whisper decoder step as OpenASR's host builds it
// for a GPU backend, restated over the ggml C API:
//   reusable one-token step graph   models/whisper/ggml_decoder_graph.rs:3869-4052
//   self attention + resident KV    ggml_decoder_graph.rs:4557-5044
//   cross attention                 ggml_decoder_graph.rs:5106-5340
//   MLP (LayerNorm, fc1, GELU, fc2) ggml_decoder_graph.rs:5342-5392
//   affine LayerNorm                ggml_decoder_graph.rs:5953-6010
//   linear with optional bias       ggml_decoder_graph.rs:5446-5490
//   cross K/V precompute            ggml_decoder_graph.rs:5780-5805
// Flash attention is on for both attentions (execution_policy.rs:21-27).

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ggml_host.h"
#include "openasr_models.h"
#include "pack_reader.h"

using oa_pack::blob;
using oa_pack::pack_reader;

extern "C" void oa_synth_normal(uint64_t seed, uint64_t stream, int64_t first, int64_t n, float mean, float std_dev,
                                float * out);

namespace {

const ggml_fp16_t kNegInf = 0xFC00;

uint64_t wh_stream(int layer, int kind) { return 700000 + (uint64_t) (layer + 1) * 1000 + (uint64_t) kind; }

std::vector<uint8_t> wh_matrix(uint64_t seed, uint64_t stream, int64_t rows, int64_t k) {
    std::vector<float> buf((size_t) (rows * k));
    oa_synth_normal(seed, stream, 0, rows * k, 0.0f, 0.02f, buf.data());
    std::vector<uint8_t> out((size_t) rows * ggml_row_size(GGML_TYPE_Q8_0, k));
    ggml_quantize_chunk(GGML_TYPE_Q8_0, buf.data(), out.data(), 0, rows, k, nullptr);
    return out;
}

std::vector<float> wh_vector(uint64_t seed, uint64_t stream, int64_t n, float mean, float std_dev) {
    std::vector<float> v((size_t) n);
    oa_synth_normal(seed, stream, 0, n, mean, std_dev, v.data());
    return v;
}

bool is_matrix(int kind) {
    return kind == OA_WH_SELF_Q || kind == OA_WH_SELF_K || kind == OA_WH_SELF_V || kind == OA_WH_SELF_O ||
           kind == OA_WH_CROSS_Q || kind == OA_WH_CROSS_K || kind == OA_WH_CROSS_V || kind == OA_WH_CROSS_O ||
           kind == OA_WH_FC1 || kind == OA_WH_FC2;
}

}  // namespace

struct oa_whisper_weights {
    oa_whisper_config cfg;
    blob tok_embd;  // synthesised, or a view into a mapped runtime pack
    std::vector<float> pos_embd, final_w, final_b;
    // per layer, indexed by oa_whisper_tensor_kind
    std::vector<std::vector<blob>> mats;
    std::vector<std::vector<std::vector<float>>> vecs;
    oa_gguf * src = nullptr;  // the mapped pack the views point into
    ~oa_whisper_weights() { oa_gguf_close(src); }
};

struct oa_whisper_model {
    oa_whisper_config cfg;
    ggml_backend_t backend;
    ggml_context * ctx;
    ggml_backend_buffer_t buf;
    ggml_tensor *tok_embd, *pos_embd, *final_w, *final_b;
    std::vector<std::vector<ggml_tensor *>> layers;  // [layer][kind]
};

namespace {

struct wh_graph {
    ggml_context * ctx = nullptr;
    ggml_cgraph * gf = nullptr;
    ggml_gallocr_t galloc = nullptr;
    ggml_tensor *token = nullptr, *pos = nullptr, *row = nullptr, *mask = nullptr, *logits = nullptr,
                *top1 = nullptr, *enc = nullptr;
    void release() {
        if (galloc) ggml_gallocr_free(galloc);
        if (ctx) ggml_free(ctx);
        *this = wh_graph();
    }
};

}  // namespace

struct oa_whisper_session {
    oa_whisper_model * m;
    int n_past = 0;
    int fa_prec = GGML_PREC_DEFAULT;  // the attentions' precision contract
    ggml_context * kv_ctx = nullptr;
    ggml_backend_buffer_t kv_buf = nullptr;
    std::vector<ggml_tensor *> k_self, v_self, k_cross, v_cross;  // per layer, f16 [d_model, positions|frames]
    wh_graph decode;
};

namespace {

// apply_affine_layer_norm: norm -> mul(w) -> add(b)
ggml_tensor * layer_norm(ggml_context * ctx, ggml_tensor * x, ggml_tensor * w, ggml_tensor * b, float eps) {
    return ggml_add(ctx, ggml_mul(ctx, ggml_norm(ctx, x, eps), w), b);
}

// apply_linear_with_optional_bias: mul_mat then add(bias)
ggml_tensor * linear(ggml_context * ctx, ggml_tensor * w, ggml_tensor * x, ggml_tensor * b) {
    ggml_tensor * y = ggml_mul_mat(ctx, w, x);
    return b ? ggml_add(ctx, y, b) : y;
}

// [hidden, T] -> [head_dim, T, heads] view for flash attention (T == 1 here)
ggml_tensor * heads_view(ggml_context * ctx, ggml_tensor * x, int hd, int heads, int T) {
    return ggml_permute(ctx, ggml_reshape_3d(ctx, x, hd, heads, T), 0, 2, 1, 3);
}

bool build_decode(oa_whisper_session * s, wh_graph & g) {
    const oa_whisper_model * m = s->m;
    const oa_whisper_config & c = m->cfg;
    const int d = c.d_model, H = c.n_head, hd = d / H, mp = c.max_positions;
    const size_t n_t = (size_t) c.n_layers * 64 + 64;
    ggml_init_params ip = {ggml_tensor_overhead() * n_t + ggml_graph_overhead_custom(n_t, false) + (1u << 16), nullptr,
                           true};
    g.ctx = ggml_init(ip);
    if (!g.ctx) return false;
    ggml_context * ctx = g.ctx;
    g.token = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 1);
    g.row = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 1);
    g.pos = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, 1);
    g.mask = ggml_new_tensor_3d(ctx, GGML_TYPE_F16, mp, 1, 1);
    ggml_set_input(g.token);
    ggml_set_input(g.row);
    ggml_set_input(g.pos);
    ggml_set_input(g.mask);
    ggml_tensor * state = ggml_add(ctx, ggml_get_rows(ctx, m->tok_embd, g.token), ggml_get_rows(ctx, m->pos_embd, g.pos));
    const float scale = 1.0f / std::sqrt((float) hd);
    const size_t row_stride = (size_t) d * 2, head_stride = (size_t) hd * 2;
    for (int l = 0; l < c.n_layers; l++) {
        const std::vector<ggml_tensor *> & L = m->layers[(size_t) l];
        // self attention (:4557-5044): K/V rows written at `row`, attention over the full span with the mask
        ggml_tensor * nrm = layer_norm(ctx, state, L[OA_WH_SELF_LN_W], L[OA_WH_SELF_LN_B], c.ln_eps);
        ggml_tensor * q = linear(ctx, L[OA_WH_SELF_Q], nrm, L[OA_WH_SELF_Q_B]);
        ggml_tensor * k = linear(ctx, L[OA_WH_SELF_K], nrm, nullptr);
        ggml_tensor * v = linear(ctx, L[OA_WH_SELF_V], nrm, L[OA_WH_SELF_V_B]);
        ggml_tensor * k_written = ggml_set_rows(ctx, s->k_self[(size_t) l], ggml_reshape_2d(ctx, k, d, 1), g.row);
        ggml_tensor * v_written = ggml_set_rows(ctx, s->v_self[(size_t) l], ggml_reshape_2d(ctx, v, d, 1), g.row);
        ggml_tensor * kc = ggml_view_3d(ctx, k_written, hd, mp, H, row_stride, head_stride, 0);
        ggml_tensor * vc = ggml_view_3d(ctx, v_written, hd, mp, H, row_stride, head_stride, 0);
        ggml_tensor * ctx_self = ggml_flash_attn_ext(ctx, heads_view(ctx, q, hd, H, 1), kc, vc, g.mask, scale, 0.0f, 0.0f);
        ggml_flash_attn_ext_set_prec(ctx_self, (ggml_prec) s->fa_prec);
        ctx_self = ggml_reshape_2d(ctx, ctx_self, d, 1);
        state = ggml_add(ctx, linear(ctx, L[OA_WH_SELF_O], ctx_self, L[OA_WH_SELF_O_B]), state);
        // cross attention (:5106-5340) over the precomputed f16 cross K/V, no mask
        nrm = layer_norm(ctx, state, L[OA_WH_CROSS_LN_W], L[OA_WH_CROSS_LN_B], c.ln_eps);
        q = linear(ctx, L[OA_WH_CROSS_Q], nrm, L[OA_WH_CROSS_Q_B]);
        ggml_tensor * ck = ggml_view_3d(ctx, s->k_cross[(size_t) l], hd, c.n_frames, H, row_stride, head_stride, 0);
        ggml_tensor * cv = ggml_view_3d(ctx, s->v_cross[(size_t) l], hd, c.n_frames, H, row_stride, head_stride, 0);
        ggml_tensor * ctx_cross = ggml_flash_attn_ext(ctx, heads_view(ctx, q, hd, H, 1), ck, cv, nullptr, scale, 0.0f, 0.0f);
        ggml_flash_attn_ext_set_prec(ctx_cross, (ggml_prec) s->fa_prec);
        ctx_cross = ggml_reshape_2d(ctx, ctx_cross, d, 1);
        state = ggml_add(ctx, linear(ctx, L[OA_WH_CROSS_O], ctx_cross, L[OA_WH_CROSS_O_B]), state);
        // MLP (:5342-5392)
        nrm = layer_norm(ctx, state, L[OA_WH_MLP_LN_W], L[OA_WH_MLP_LN_B], c.ln_eps);
        ggml_tensor * h = linear(ctx, L[OA_WH_FC1], nrm, L[OA_WH_FC1_B]);
        switch (c.ffn_act) {  // nn/decoder.rs:1125-1138
            case 1: h = ggml_relu(ctx, h); break;
            case 2: h = ggml_gelu_erf(ctx, h); break;
            case 3: h = ggml_silu(ctx, h); break;
            default: h = ggml_gelu(ctx, h); break;
        }
        state = ggml_add(ctx, linear(ctx, L[OA_WH_FC2], h, L[OA_WH_FC2_B]), state);
    }
    ggml_tensor * nrm = layer_norm(ctx, state, m->final_w, m->final_b, c.ln_eps);
    g.logits = ggml_mul_mat(ctx, m->tok_embd, nrm);  // output projection tied to the token embedding
    g.top1 = ggml_argmax_first(ctx, g.logits);
    ggml_set_output(g.logits);
    ggml_set_output(g.top1);
    g.gf = ggml_new_graph_custom(ctx, n_t, false);
    ggml_build_forward_expand(g.gf, g.top1);
    g.galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m->backend));
    return ggml_gallocr_alloc_graph(g.galloc, g.gf);
}

}  // namespace

extern "C" {

oa_whisper_weights * oa_whisper_weights_synthesize(const oa_whisper_config * cfg) {
    const oa_whisper_config & c = *cfg;
    oa_whisper_weights * w = new oa_whisper_weights;
    w->cfg = c;
    const int d = c.d_model;
    w->tok_embd = wh_matrix(c.seed, wh_stream(-1, OA_WH_TOKEN_EMBD), c.vocab, d);
    w->pos_embd = wh_vector(c.seed, wh_stream(-1, OA_WH_POS_EMBD), (int64_t) c.max_positions * d, 0.0f, 0.02f);
    w->final_w = wh_vector(c.seed, wh_stream(-1, OA_WH_FINAL_LN_W), d, 1.0f, 0.05f);
    w->final_b = wh_vector(c.seed, wh_stream(-1, OA_WH_FINAL_LN_B), d, 0.0f, 0.02f);
    w->mats.assign((size_t) c.n_layers, std::vector<blob>(OA_WH_LAYER_KINDS));
    w->vecs.assign((size_t) c.n_layers, std::vector<std::vector<float>>(OA_WH_LAYER_KINDS));
    for (int l = 0; l < c.n_layers; l++) {
        for (int kind = 0; kind < OA_WH_LAYER_KINDS; kind++) {
            const uint64_t st = wh_stream(l, kind);
            if (is_matrix(kind)) {
                const int64_t rows = kind == OA_WH_FC1 ? c.ffn : d;
                const int64_t k = kind == OA_WH_FC2 ? c.ffn : d;
                w->mats[(size_t) l][(size_t) kind] = wh_matrix(c.seed, st, rows, k);
            } else {
                const bool ln_w = kind == OA_WH_SELF_LN_W || kind == OA_WH_CROSS_LN_W || kind == OA_WH_MLP_LN_W;
                const int64_t n = kind == OA_WH_FC1_B ? c.ffn : d;
                w->vecs[(size_t) l][(size_t) kind] = wh_vector(c.seed, st, n, ln_w ? 1.0f : 0.0f, ln_w ? 0.05f : 0.02f);
            }
        }
    }
    return w;
}

void oa_whisper_weights_free(oa_whisper_weights * w) { delete w; }

const void * oa_whisper_weights_tensor(const oa_whisper_weights * w, int layer, int kind, size_t * nbytes) {
    auto u8 = [&](const blob & v) -> const void * {
        if (nbytes) *nbytes = v.size();
        return v.data();
    };
    auto f = [&](const std::vector<float> & v) -> const void * {
        if (nbytes) *nbytes = v.size() * sizeof(float);
        return v.data();
    };
    switch (kind) {
        case OA_WH_TOKEN_EMBD: return u8(w->tok_embd);
        case OA_WH_POS_EMBD: return f(w->pos_embd);
        case OA_WH_FINAL_LN_W: return f(w->final_w);
        case OA_WH_FINAL_LN_B: return f(w->final_b);
        default: break;
    }
    if (layer < 0 || layer >= w->cfg.n_layers || kind < 0 || kind >= OA_WH_LAYER_KINDS) return nullptr;
    return is_matrix(kind) ? u8(w->mats[(size_t) layer][(size_t) kind]) : f(w->vecs[(size_t) layer][(size_t) kind]);
}

// A whisper runtime pack (.oasr v1 = GGUF): hparams under whisper.* (the
// keys of models/whisper/runtime_contract.rs:180-230), decoder tensors under
// the names of models/whisper/ggml_tensor_binding.rs:135-210, matrices Q8_0
// bound as views into the mapping, vectors and the positional table copied.
oa_whisper_weights * oa_whisper_weights_load_gguf(const char * path, char * err, size_t err_cap) {
    auto report = [&](const std::string & msg) -> oa_whisper_weights * {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", msg.c_str());
        return nullptr;
    };
    char gerr[256] = {0};
    oa_gguf * g = oa_gguf_open(path, gerr, sizeof(gerr));
    if (!g) return report(gerr);
    oa_whisper_weights * w = new oa_whisper_weights;
    w->src = g;
    pack_reader r{g, {}};
    auto bad = [&](const std::string & msg) {
        delete w;
        return report(msg);
    };
    if (const char * v = oa_gguf_get_str(g, "openasr.package.version"); v && std::strcmp(v, "1") != 0)
        return bad(std::string("unsupported openasr.package.version ") + v);
    if (const char * a = oa_gguf_get_str(g, "general.architecture"); a && std::strcmp(a, "whisper") != 0)
        return bad(std::string("general.architecture is ") + a + ", not whisper");
    oa_whisper_config & c = w->cfg;
    c = oa_whisper_config{};
    if (!r.key_i("whisper.decoder.block_count", c.n_layers) || !r.key_i("whisper.decoder.embedding_length", c.d_model) ||
        !r.key_i("whisper.decoder.attention.head_count", c.n_head) ||
        !r.key_i("whisper.decoder.context_length", c.max_positions) || !r.key_i("whisper.vocab_size", c.vocab) ||
        !r.key_i("whisper.encoder.context_length", c.n_frames))
        return bad(r.err);
    if (c.d_model % c.n_head != 0) return bad("embedding_length is not a multiple of head_count");
    if (c.d_model % 32 != 0) return bad("embedding_length is not a multiple of the Q8_0 block");
    c.ln_eps = 1e-5f;
    c.seed = 0;
    const int64_t fi = oa_gguf_find_tensor(g, "decoder.layers.0.fc1.weight");
    if (fi < 0) return bad("missing tensor decoder.layers.0.fc1.weight");
    int ft = 0;
    int64_t ne[4];
    oa_gguf_tensor_info(g, fi, &ft, ne);
    c.ffn = (int) ne[1];
    const int d = c.d_model;
    if (!r.mat("decoder.token_embedding.weight", d, c.vocab, GGML_TYPE_Q8_0, w->tok_embd) ||
        !r.vec("decoder.positional_embedding", d, w->pos_embd, c.max_positions) ||
        !r.vec("decoder.layer_norm.weight", d, w->final_w) || !r.vec("decoder.layer_norm.bias", d, w->final_b))
        return bad(r.err);
    w->mats.assign((size_t) c.n_layers, std::vector<blob>(OA_WH_LAYER_KINDS));
    w->vecs.assign((size_t) c.n_layers, std::vector<std::vector<float>>(OA_WH_LAYER_KINDS));
    static const struct {
        int kind;
        const char * name;
    } names[] = {
        {OA_WH_SELF_LN_W, "self_attn_layer_norm.weight"}, {OA_WH_SELF_LN_B, "self_attn_layer_norm.bias"},
        {OA_WH_SELF_Q, "self_attn.q_proj.weight"},        {OA_WH_SELF_Q_B, "self_attn.q_proj.bias"},
        {OA_WH_SELF_K, "self_attn.k_proj.weight"},        {OA_WH_SELF_V, "self_attn.v_proj.weight"},
        {OA_WH_SELF_V_B, "self_attn.v_proj.bias"},        {OA_WH_SELF_O, "self_attn.out_proj.weight"},
        {OA_WH_SELF_O_B, "self_attn.out_proj.bias"},      {OA_WH_CROSS_LN_W, "encoder_attn_layer_norm.weight"},
        {OA_WH_CROSS_LN_B, "encoder_attn_layer_norm.bias"}, {OA_WH_CROSS_Q, "cross_attn.q_proj.weight"},
        {OA_WH_CROSS_Q_B, "cross_attn.q_proj.bias"},      {OA_WH_CROSS_K, "cross_attn.k_proj.weight"},
        {OA_WH_CROSS_V, "cross_attn.v_proj.weight"},      {OA_WH_CROSS_V_B, "cross_attn.v_proj.bias"},
        {OA_WH_CROSS_O, "cross_attn.out_proj.weight"},    {OA_WH_CROSS_O_B, "cross_attn.out_proj.bias"},
        {OA_WH_MLP_LN_W, "final_layer_norm.weight"},      {OA_WH_MLP_LN_B, "final_layer_norm.bias"},
        {OA_WH_FC1, "fc1.weight"},                        {OA_WH_FC1_B, "fc1.bias"},
        {OA_WH_FC2, "fc2.weight"},                        {OA_WH_FC2_B, "fc2.bias"},
    };
    for (int l = 0; l < c.n_layers; l++) {
        const std::string p = "decoder.layers." + std::to_string(l) + ".";
        for (const auto & n : names) {
            const int kind = n.kind;
            bool ok;
            if (is_matrix(kind)) {
                const int64_t rows = kind == OA_WH_FC1 ? c.ffn : d;
                const int64_t k = kind == OA_WH_FC2 ? c.ffn : d;
                ok = r.mat(p + n.name, k, rows, GGML_TYPE_Q8_0, w->mats[(size_t) l][(size_t) kind]);
            } else {
                ok = r.vec(p + n.name, kind == OA_WH_FC1_B ? c.ffn : d, w->vecs[(size_t) l][(size_t) kind]);
            }
            if (!ok) return bad(r.err);
        }
    }
    return w;
}

void oa_whisper_weights_config(const oa_whisper_weights * w, oa_whisper_config * out) { *out = w->cfg; }

oa_whisper_model * oa_whisper_model_create(ggml_backend_t backend, const oa_whisper_weights * w) {
    const oa_whisper_config & c = w->cfg;
    oa_whisper_model * m = new oa_whisper_model;
    m->cfg = c;
    m->backend = backend;
    ggml_init_params ip = {ggml_tensor_overhead() * ((size_t) c.n_layers * OA_WH_LAYER_KINDS + 16), nullptr, true};
    m->ctx = ggml_init(ip);
    const int d = c.d_model;
    m->tok_embd = ggml_new_tensor_2d(m->ctx, GGML_TYPE_Q8_0, d, c.vocab);
    m->pos_embd = ggml_new_tensor_2d(m->ctx, GGML_TYPE_F32, d, c.max_positions);
    m->final_w = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, d);
    m->final_b = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, d);
    m->layers.assign((size_t) c.n_layers, std::vector<ggml_tensor *>(OA_WH_LAYER_KINDS, nullptr));
    for (int l = 0; l < c.n_layers; l++) {
        for (int kind = 0; kind < OA_WH_LAYER_KINDS; kind++) {
            ggml_tensor *& t = m->layers[(size_t) l][(size_t) kind];
            if (is_matrix(kind)) {
                const int64_t rows = kind == OA_WH_FC1 ? c.ffn : d;
                const int64_t k = kind == OA_WH_FC2 ? c.ffn : d;
                t = ggml_new_tensor_2d(m->ctx, GGML_TYPE_Q8_0, k, rows);
            } else {
                t = ggml_new_tensor_1d(m->ctx, GGML_TYPE_F32, kind == OA_WH_FC1_B ? c.ffn : d);
            }
        }
    }
    m->buf = ggml_backend_alloc_ctx_tensors_from_buft(m->ctx, ggml_backend_get_default_buffer_type(backend));
    if (!m->buf) {
        ggml_free(m->ctx);
        delete m;
        return nullptr;
    }
    ggml_backend_buffer_set_usage(m->buf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    ggml_backend_tensor_set(m->tok_embd, w->tok_embd.data(), 0, w->tok_embd.size());
    ggml_backend_tensor_set(m->pos_embd, w->pos_embd.data(), 0, w->pos_embd.size() * 4);
    ggml_backend_tensor_set(m->final_w, w->final_w.data(), 0, w->final_w.size() * 4);
    ggml_backend_tensor_set(m->final_b, w->final_b.data(), 0, w->final_b.size() * 4);
    for (int l = 0; l < c.n_layers; l++) {
        for (int kind = 0; kind < OA_WH_LAYER_KINDS; kind++) {
            size_t n = 0;
            const void * src = oa_whisper_weights_tensor(w, l, kind, &n);
            ggml_backend_tensor_set(m->layers[(size_t) l][(size_t) kind], src, 0, n);
        }
    }
    return m;
}

void oa_whisper_model_free(oa_whisper_model * m) {
    if (!m) return;
    ggml_backend_buffer_free(m->buf);
    ggml_free(m->ctx);
    delete m;
}

oa_whisper_session * oa_whisper_session_create(oa_whisper_model * m) {
    const oa_whisper_config & c = m->cfg;
    oa_whisper_session * s = new oa_whisper_session;
    s->m = m;
    ggml_init_params ip = {ggml_tensor_overhead() * ((size_t) c.n_layers * 4 + 4), nullptr, true};
    s->kv_ctx = ggml_init(ip);
    for (int l = 0; l < c.n_layers; l++) {
        s->k_self.push_back(ggml_new_tensor_2d(s->kv_ctx, GGML_TYPE_F16, c.d_model, c.max_positions));
        s->v_self.push_back(ggml_new_tensor_2d(s->kv_ctx, GGML_TYPE_F16, c.d_model, c.max_positions));
        s->k_cross.push_back(ggml_new_tensor_2d(s->kv_ctx, GGML_TYPE_F16, c.d_model, c.n_frames));
        s->v_cross.push_back(ggml_new_tensor_2d(s->kv_ctx, GGML_TYPE_F16, c.d_model, c.n_frames));
    }
    s->kv_buf = ggml_backend_alloc_ctx_tensors_from_buft(s->kv_ctx, ggml_backend_get_default_buffer_type(m->backend));
    if (!s->kv_buf) {
        ggml_free(s->kv_ctx);
        delete s;
        return nullptr;
    }
    ggml_backend_buffer_clear(s->kv_buf, 0);
    return s;
}

void oa_whisper_session_free(oa_whisper_session * s) {
    if (!s) return;
    s->decode.release();
    ggml_backend_buffer_free(s->kv_buf);
    ggml_free(s->kv_ctx);
    delete s;
}

int oa_whisper_session_position(const oa_whisper_session * s) { return s->n_past; }

int oa_whisper_session_set_flash_attention_precision(oa_whisper_session * s, int precision) {
    if (precision != GGML_PREC_DEFAULT && precision != GGML_PREC_F32) return GGML_STATUS_FAILED;
    if (precision != s->fa_prec) {
        s->fa_prec = precision;
        s->decode.release();  // rebuilt under the new contract on the next step
    }
    return GGML_STATUS_SUCCESS;
}

int oa_whisper_set_encoder(oa_whisper_session * s, const float * enc) {
    const oa_whisper_model * m = s->m;
    const oa_whisper_config & c = m->cfg;
    const size_t n_t = (size_t) c.n_layers * 8 + 16;
    ggml_init_params ip = {ggml_tensor_overhead() * n_t + ggml_graph_overhead_custom(n_t, false) + (1u << 16), nullptr,
                           true};
    wh_graph g;
    g.ctx = ggml_init(ip);
    if (!g.ctx) return GGML_STATUS_ALLOC_FAILED;
    g.enc = ggml_new_tensor_2d(g.ctx, GGML_TYPE_F32, c.d_model, c.n_frames);
    ggml_set_input(g.enc);
    g.gf = ggml_new_graph_custom(g.ctx, n_t, false);
    for (int l = 0; l < c.n_layers; l++) {
        const std::vector<ggml_tensor *> & L = m->layers[(size_t) l];
        ggml_tensor * kk = ggml_mul_mat(g.ctx, L[OA_WH_CROSS_K], g.enc);
        ggml_tensor * vv = ggml_add(g.ctx, ggml_mul_mat(g.ctx, L[OA_WH_CROSS_V], g.enc), L[OA_WH_CROSS_V_B]);
        ggml_build_forward_expand(g.gf, ggml_cpy(g.ctx, kk, s->k_cross[(size_t) l]));
        ggml_build_forward_expand(g.gf, ggml_cpy(g.ctx, vv, s->v_cross[(size_t) l]));
    }
    g.galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(m->backend));
    if (!ggml_gallocr_alloc_graph(g.galloc, g.gf)) {
        g.release();
        return GGML_STATUS_ALLOC_FAILED;
    }
    ggml_backend_tensor_set(g.enc, enc, 0, (size_t) c.d_model * c.n_frames * sizeof(float));
    const int st = ggml_backend_graph_compute(m->backend, g.gf);
    g.release();
    return st;
}

int oa_whisper_decode_step(oa_whisper_session * s, int32_t token, int32_t * top1_out, float * logits_out) {
    const oa_whisper_config & c = s->m->cfg;
    if (s->n_past >= c.max_positions) return GGML_STATUS_FAILED;
    if (!s->decode.gf && !build_decode(s, s->decode)) {
        s->decode.release();
        return GGML_STATUS_ALLOC_FAILED;
    }
    wh_graph & g = s->decode;
    const int32_t p = s->n_past;
    std::vector<ggml_fp16_t> mask((size_t) c.max_positions, kNegInf);
    for (int j = 0; j <= p; j++) mask[(size_t) j] = 0;
    ggml_backend_tensor_set(g.token, &token, 0, 4);
    ggml_backend_tensor_set(g.row, &p, 0, 4);
    ggml_backend_tensor_set(g.pos, &p, 0, 4);
    ggml_backend_tensor_set(g.mask, mask.data(), 0, mask.size() * 2);
    const int st = ggml_backend_graph_compute(s->m->backend, g.gf);
    if (st != GGML_STATUS_SUCCESS) return st;
    s->n_past++;
    if (top1_out) ggml_backend_tensor_get(g.top1, top1_out, 0, 4);
    if (logits_out) ggml_backend_tensor_get(g.logits, logits_out, 0, (size_t) c.vocab * 4);
    return GGML_STATUS_SUCCESS;
}

int oa_whisper_generate(oa_whisper_session * s, int32_t first_token, int n_steps, int32_t * out_tokens,
                        double * step_ms) {
    int32_t cur = first_token;
    for (int i = 0; i < n_steps; i++) {
        const auto t0 = std::chrono::steady_clock::now();
        const int st = oa_whisper_decode_step(s, cur, &out_tokens[i], nullptr);
        if (step_ms) step_ms[i] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        if (st != GGML_STATUS_SUCCESS) return st;
        cur = out_tokens[i];
    }
    return GGML_STATUS_SUCCESS;
}

int oa_whisper_read_cross(const oa_whisper_session * s, int layer, uint16_t * k_out, uint16_t * v_out) {
    const oa_whisper_config & c = s->m->cfg;
    const size_t n = (size_t) c.d_model * c.n_frames * 2;
    if (k_out && ggml_backend_tensor_get(s->k_cross[(size_t) layer], k_out, 0, n)) return 1;
    if (v_out && ggml_backend_tensor_get(s->v_cross[(size_t) layer], v_out, 0, n)) return 1;
    return 0;
}

int oa_whisper_read_self(const oa_whisper_session * s, int layer, uint16_t * k_out, uint16_t * v_out) {
    const oa_whisper_config & c = s->m->cfg;
    if (layer < 0 || layer >= c.n_layers) return 1;
    const size_t n = (size_t) c.d_model * c.max_positions * 2;
    if (k_out && ggml_backend_tensor_get(s->k_self[(size_t) layer], k_out, 0, n)) return 1;
    if (v_out && ggml_backend_tensor_get(s->v_self[(size_t) layer], v_out, 0, n)) return 1;
    return 0;
}

struct ggml_cgraph * oa_whisper_decode_graph(oa_whisper_session * s) { return s->decode.gf; }

}  // extern "C"
