// qwen_audio_encoder.cpp -- the Qwen3-ASR audio encoder (the decoder's prefix
// producer) as OpenASR's host builds its graph for a GPU backend, restated
// over the ggml C API:
//   mel chunk layout, positions, mask       models/qwen/audio_encoder.rs:324-360, 798-845
//   conv stem (3 x conv_2d + bias + GELU_ERF) audio_encoder.rs:480-552, nn/conv.rs:39-52, 82-111
//   channel permute, conv_out, positions    audio_encoder.rs:553-605
//   sinusoidal position table               nn/encoder.rs:575-610
//   encoder block (pre-norm, flash attention over strided head views, GELU_ERF FFN)
//                                           nn/encoder.rs:654-870, nn/attn.rs:89-126,
//                                           nn/norm.rs:10-31, nn/ffn.rs:22-50
//   ln_post, proj1, GELU_ERF, proj2         audio_encoder.rs:615-672
// The weights are synthesised (seeded) or read from a qwen3-asr runtime pack
// (load_qwen3_audio_encoder_weights_from_reader, audio_encoder.rs:896-1050);
// the graph is the same op sequence whatever their source.

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "ggml_host.h"
#include "openasr_models.h"
#include "pack_reader.h"

extern "C" void oa_synth_normal(uint64_t seed, uint64_t stream, int64_t first, int64_t n, float mean, float std_dev,
                                float * out);

namespace {

constexpr int kChunkFrames = 100;  // QWEN3_AUDIO_CHUNK_FRAMES (audio_encoder.rs:52)
constexpr float kLnEps = 1.0e-5f;  // QWEN3_AUDIO_LAYER_NORM_EPSILON (:53)

// floor((n + 2 p - d (k - 1) - 1) / s) + 1 with k 3, s 2, p 1, d 1 (runtime_contract.rs:29-45)
int conv_out_len(int n) { return (n - 1) / 2 + 1; }

uint64_t qa_stream(int layer, int kind) { return 900000 + (uint64_t) (layer + 1) * 1000 + (uint64_t) kind; }

bool is_layer_matrix(int kind) {
    return kind == OA_QA_Q || kind == OA_QA_K || kind == OA_QA_V || kind == OA_QA_O || kind == OA_QA_UP ||
           kind == OA_QA_DOWN;
}

std::vector<float> normal(uint64_t seed, uint64_t stream, int64_t n, float mean, float std_dev) {
    std::vector<float> v((size_t) n);
    oa_synth_normal(seed, stream, 0, n, mean, std_dev, v.data());
    return v;
}

// [rows][k] matrix of N(0, 0.02) values in the projection type
std::vector<uint8_t> matrix(int wtype, uint64_t seed, uint64_t stream, int64_t rows, int64_t k) {
    const std::vector<float> f = normal(seed, stream, rows * k, 0.0f, 0.02f);
    std::vector<uint8_t> out((size_t) rows * ggml_row_size((ggml_type) wtype, k));
    ggml_quantize_chunk((ggml_type) wtype, f.data(), out.data(), 0, rows, k, nullptr);
    return out;
}

std::vector<uint8_t> bytes_of(const std::vector<float> & v) {
    std::vector<uint8_t> b(v.size() * 4);
    std::memcpy(b.data(), v.data(), b.size());
    return b;
}

}  // namespace

struct oa_qwen_audio_weights {
    oa_qwen_audio_config cfg;
    int freq_bins;                                  // mel bins after the three convolutions
    bool conv_out_bias = true;                      // optional in a pack (audio_encoder.rs:907-915)
    std::map<int, std::vector<uint8_t>> global;     // kind -> bytes
    std::vector<std::vector<std::vector<uint8_t>>> layers;  // [layer][kind]
};

struct oa_qwen_audio_encoder {
    oa_qwen_audio_config cfg;
    int freq_bins;
    bool conv_out_bias;
    ggml_backend_t backend;
    ggml_context * ctx = nullptr;
    ggml_backend_buffer_t buf = nullptr;
    std::map<int, ggml_tensor *> g;                // global weights
    std::vector<std::vector<ggml_tensor *>> L;     // [layer][kind]
    // the self-attention's flash-attention precision (GGML_PREC_DEFAULT as
    // the reference builds it, or GGML_PREC_F32)
    int fa_prec = GGML_PREC_DEFAULT;
    // the graph of the last chunk count
    int graph_chunks = 0;
    ggml_context * gctx = nullptr;
    ggml_cgraph * gf = nullptr;
    ggml_gallocr_t galloc = nullptr;
    ggml_tensor *mel = nullptr, *pos = nullptr, *mask = nullptr, *out = nullptr;
    void release_graph() {
        if (galloc) ggml_gallocr_free(galloc);
        if (gctx) ggml_free(gctx);
        galloc = nullptr;
        gctx = nullptr;
        gf = nullptr;
        graph_chunks = 0;
    }
};

namespace {

// apply_affine_layer_norm (nn/norm.rs:10-31): norm -> mul(w) -> add(b)
ggml_tensor * layer_norm(ggml_context * ctx, ggml_tensor * x, ggml_tensor * w, ggml_tensor * b) {
    return ggml_add(ctx, ggml_mul(ctx, ggml_norm(ctx, x, kLnEps), w), b);
}

// linear_with_bias (nn/encoder.rs:655-671): mul_mat then add(bias)
ggml_tensor * linear(ggml_context * ctx, ggml_tensor * w, ggml_tensor * x, ggml_tensor * b) {
    return ggml_add(ctx, ggml_mul_mat(ctx, w, x), b);
}

// reshape_projection_to_attention_heads without the CONT (strided views on a
// GPU-class backend, nn/encoder.rs:735-790): [hd * heads, T] -> [hd, T, heads]
ggml_tensor * heads_view(ggml_context * ctx, ggml_tensor * x, int hd, int heads, int T) {
    return ggml_permute(ctx, ggml_reshape_3d(ctx, x, hd, heads, T), 0, 2, 1, 3);
}

// transformer_layer (nn/encoder.rs:678-870) with flash attention and GELU_ERF
ggml_tensor * encoder_layer(ggml_context * ctx, ggml_tensor * x, ggml_tensor * mask16,
                            const std::vector<ggml_tensor *> & W, const oa_qwen_audio_config & c, int rows,
                            int fa_prec) {
    const int hd = c.d_model / c.n_heads;
    ggml_tensor * residual = x;
    ggml_tensor * h = layer_norm(ctx, x, W[OA_QA_ATTN_NORM_W], W[OA_QA_ATTN_NORM_B]);
    ggml_tensor * q = linear(ctx, W[OA_QA_Q], h, W[OA_QA_Q_B]);
    ggml_tensor * k = linear(ctx, W[OA_QA_K], h, W[OA_QA_K_B]);
    ggml_tensor * v = linear(ctx, W[OA_QA_V], h, W[OA_QA_V_B]);
    const float scale = 1.0f / std::sqrt((float) hd);
    ggml_tensor * att = ggml_flash_attn_ext(ctx, heads_view(ctx, q, hd, c.n_heads, rows),
                                            heads_view(ctx, k, hd, c.n_heads, rows),
                                            heads_view(ctx, v, hd, c.n_heads, rows), mask16, scale, 0.0f, 0.0f);
    ggml_flash_attn_ext_set_prec(att, (ggml_prec) fa_prec);
    att = ggml_reshape_2d(ctx, att, (int64_t) hd * c.n_heads, rows);
    x = ggml_add(ctx, linear(ctx, W[OA_QA_O], att, W[OA_QA_O_B]), residual);
    // FFN (nn/ffn.rs:22-50): up, GELU_ERF, down, residual
    residual = x;
    h = layer_norm(ctx, x, W[OA_QA_FFN_NORM_W], W[OA_QA_FFN_NORM_B]);
    h = ggml_gelu_erf(ctx, linear(ctx, W[OA_QA_UP], h, W[OA_QA_UP_B]));
    return ggml_add(ctx, linear(ctx, W[OA_QA_DOWN], h, W[OA_QA_DOWN_B]), residual);
}

bool build_graph(oa_qwen_audio_encoder * e, int chunks) {
    const oa_qwen_audio_config & c = e->cfg;
    const int cof = conv_out_len(conv_out_len(conv_out_len(kChunkFrames)));
    const int rows = chunks * cof;
    ggml_init_params ip = {ggml_tensor_overhead() * ((size_t) c.n_layers * 64 + 256) + ggml_graph_overhead_custom(8192, false),
                           nullptr, true};
    e->gctx = ggml_init(ip);
    if (!e->gctx) return false;
    ggml_context * ctx = e->gctx;
    e->mel = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, kChunkFrames, c.n_mels, 1, chunks);
    e->pos = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 1, cof);
    e->mask = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, rows, rows);
    ggml_set_input(e->mel);
    ggml_set_input(e->pos);
    ggml_set_input(e->mask);
    // sinusoidal positions, half-split channels (nn/encoder.rs:575-590)
    ggml_tensor * ang = ggml_mul_mat(ctx, e->g[OA_QA_INV_TIMESCALES], e->pos);
    ggml_tensor * posemb = ggml_concat(ctx, ggml_sin(ctx, ang), ggml_cos(ctx, ang), 0);
    // conv stem: [W time, H mel, C, chunk] -> ... (stride 2, pad 1, dilation 1)
    ggml_tensor * x = e->mel;
    const int conv_w[3] = {OA_QA_CONV1_W, OA_QA_CONV2_W, OA_QA_CONV3_W};
    for (int i = 0; i < 3; i++) {
        ggml_tensor * b4 = ggml_reshape_4d(ctx, e->g[conv_w[i] + 1], 1, 1, c.conv_channels, 1);  // nn/conv.rs:39-52
        x = ggml_gelu_erf(ctx, ggml_add(ctx, ggml_conv_2d(ctx, e->g[conv_w[i]], x, 2, 2, 1, 1, 1, 1), b4));
    }
    // [cof, F, C, chunks] -> [F, C, cof, chunks] -> [C F, cof, chunks]
    x = ggml_cont(ctx, ggml_permute(ctx, x, 2, 0, 1, 3));
    x = ggml_reshape_3d(ctx, x, (int64_t) c.conv_channels * e->freq_bins, cof, chunks);
    x = ggml_mul_mat(ctx, e->g[OA_QA_CONV_OUT], x);
    if (e->conv_out_bias) x = ggml_add(ctx, x, e->g[OA_QA_CONV_OUT_B]);
    x = ggml_add(ctx, x, posemb);
    x = ggml_reshape_2d(ctx, x, c.d_model, rows);
    // flash attention takes an f16 mask: the f32 one cast once per layer (nn/encoder.rs:794-800)
    for (int l = 0; l < c.n_layers; l++) {
        ggml_tensor * mask16 = ggml_cast(ctx, e->mask, GGML_TYPE_F16);
        x = encoder_layer(ctx, x, mask16, e->L[(size_t) l], c, rows, e->fa_prec);
    }
    x = layer_norm(ctx, x, e->g[OA_QA_LN_POST_W], e->g[OA_QA_LN_POST_B]);
    x = ggml_gelu_erf(ctx, linear(ctx, e->g[OA_QA_PROJ1], x, e->g[OA_QA_PROJ1_B]));
    e->out = linear(ctx, e->g[OA_QA_PROJ2], x, e->g[OA_QA_PROJ2_B]);
    ggml_set_output(e->out);
    e->gf = ggml_new_graph_custom(ctx, 8192, false);
    ggml_build_forward_expand(e->gf, e->out);
    e->galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(e->backend));
    if (!ggml_gallocr_alloc_graph(e->galloc, e->gf)) return false;
    e->graph_chunks = chunks;
    return true;
}

}  // namespace

extern "C" {

int oa_qwen_audio_token_count(int n_frames) {
    if (n_frames <= 0) return 0;
    const int chunks = (n_frames + kChunkFrames - 1) / kChunkFrames;
    return chunks * conv_out_len(conv_out_len(conv_out_len(kChunkFrames)));
}

oa_qwen_audio_weights * oa_qwen_audio_weights_synthesize(const oa_qwen_audio_config * cfg) {
    const oa_qwen_audio_config & c = *cfg;
    if (c.n_mels < 8 || c.conv_channels < 1 || c.d_model < 2 || c.d_model % 2 || c.n_heads < 1 ||
        c.d_model % c.n_heads || c.n_layers < 0 || c.ffn < 1 || c.out_dim < 1)
        return nullptr;
    if (c.wtype != GGML_TYPE_F32 && c.wtype != GGML_TYPE_F16 && c.wtype != GGML_TYPE_Q8_0) return nullptr;
    oa_qwen_audio_weights * w = new oa_qwen_audio_weights;
    w->cfg = c;
    w->freq_bins = conv_out_len(conv_out_len(conv_out_len(c.n_mels)));
    const int64_t ck = (int64_t) c.conv_channels * w->freq_bins;
    if (c.wtype == GGML_TYPE_Q8_0 && (ck % 32 || c.d_model % 32 || c.ffn % 32)) {
        delete w;
        return nullptr;
    }
    const uint64_t s = c.seed;
    const int C = c.conv_channels, d = c.d_model;
    // conv kernels [OC][IC][3][3] f32, scaled to keep unit-order activations
    w->global[OA_QA_CONV1_W] = bytes_of(normal(s, qa_stream(-1, OA_QA_CONV1_W), (int64_t) C * 9, 0.0f, 0.3f));
    w->global[OA_QA_CONV2_W] =
        bytes_of(normal(s, qa_stream(-1, OA_QA_CONV2_W), (int64_t) C * C * 9, 0.0f, 1.0f / std::sqrt(9.0f * C)));
    w->global[OA_QA_CONV3_W] =
        bytes_of(normal(s, qa_stream(-1, OA_QA_CONV3_W), (int64_t) C * C * 9, 0.0f, 1.0f / std::sqrt(9.0f * C)));
    for (int kind : {OA_QA_CONV1_B, OA_QA_CONV2_B, OA_QA_CONV3_B})
        w->global[kind] = bytes_of(normal(s, qa_stream(-1, kind), C, 0.0f, 0.02f));
    w->global[OA_QA_CONV_OUT] = matrix(c.wtype, s, qa_stream(-1, OA_QA_CONV_OUT), d, ck);
    w->global[OA_QA_CONV_OUT_B] = bytes_of(normal(s, qa_stream(-1, OA_QA_CONV_OUT_B), d, 0.0f, 0.02f));
    w->global[OA_QA_LN_POST_W] = bytes_of(normal(s, qa_stream(-1, OA_QA_LN_POST_W), d, 1.0f, 0.05f));
    w->global[OA_QA_LN_POST_B] = bytes_of(normal(s, qa_stream(-1, OA_QA_LN_POST_B), d, 0.0f, 0.02f));
    w->global[OA_QA_PROJ1] = matrix(c.wtype, s, qa_stream(-1, OA_QA_PROJ1), d, d);
    w->global[OA_QA_PROJ1_B] = bytes_of(normal(s, qa_stream(-1, OA_QA_PROJ1_B), d, 0.0f, 0.02f));
    w->global[OA_QA_PROJ2] = matrix(c.wtype, s, qa_stream(-1, OA_QA_PROJ2), c.out_dim, d);
    w->global[OA_QA_PROJ2_B] = bytes_of(normal(s, qa_stream(-1, OA_QA_PROJ2_B), c.out_dim, 0.0f, 0.02f));
    // half_split_position_inverse_timescales (nn/encoder.rs:604-610)
    const int half = d / 2;
    const float log_inc = std::log(10000.0f) / (float) (half - 1 > 1 ? half - 1 : 1);
    std::vector<float> inv((size_t) half);
    for (int i = 0; i < half; i++) inv[(size_t) i] = std::exp(-log_inc * (float) i);
    w->global[OA_QA_INV_TIMESCALES] = bytes_of(inv);
    w->layers.assign((size_t) c.n_layers, std::vector<std::vector<uint8_t>>(OA_QA_LAYER_KINDS));
    for (int l = 0; l < c.n_layers; l++) {
        auto & L = w->layers[(size_t) l];
        for (int kind = 0; kind < OA_QA_LAYER_KINDS; kind++) {
            const uint64_t st = qa_stream(l, kind);
            if (is_layer_matrix(kind)) {
                const int64_t rows = kind == OA_QA_UP ? c.ffn : d;
                const int64_t k = kind == OA_QA_DOWN ? c.ffn : d;
                L[(size_t) kind] = matrix(c.wtype, s, st, rows, k);
            } else {
                const bool norm_w = kind == OA_QA_ATTN_NORM_W || kind == OA_QA_FFN_NORM_W;
                L[(size_t) kind] = bytes_of(normal(s, st, kind == OA_QA_UP_B ? c.ffn : d, norm_w ? 1.0f : 0.0f,
                                                   norm_w ? 0.05f : 0.02f));
            }
        }
    }
    return w;
}

void oa_qwen_audio_weights_free(oa_qwen_audio_weights * w) { delete w; }

const void * oa_qwen_audio_weights_tensor(const oa_qwen_audio_weights * w, int layer, int kind, size_t * nbytes) {
    const std::vector<uint8_t> * b = nullptr;
    if (layer < 0) {
        auto it = w->global.find(kind);
        if (it != w->global.end()) b = &it->second;
    } else if (layer < w->cfg.n_layers && kind >= 0 && kind < OA_QA_LAYER_KINDS) {
        b = &w->layers[(size_t) layer][(size_t) kind];
    }
    if (nbytes) *nbytes = b ? b->size() : 0;
    return b ? b->data() : nullptr;
}

oa_qwen_audio_encoder * oa_qwen_audio_encoder_create(ggml_backend_t backend, const oa_qwen_audio_weights * w) {
    const oa_qwen_audio_config & c = w->cfg;
    oa_qwen_audio_encoder * e = new oa_qwen_audio_encoder;
    e->cfg = c;
    e->freq_bins = w->freq_bins;
    e->conv_out_bias = w->conv_out_bias;
    e->backend = backend;
    ggml_init_params ip = {ggml_tensor_overhead() * ((size_t) c.n_layers * OA_QA_LAYER_KINDS + 32), nullptr, true};
    e->ctx = ggml_init(ip);
    const int C = c.conv_channels, d = c.d_model;
    const ggml_type wt = (ggml_type) c.wtype;
    const int64_t ck = (int64_t) C * w->freq_bins;
    e->g[OA_QA_CONV1_W] = ggml_new_tensor_4d(e->ctx, GGML_TYPE_F32, 3, 3, 1, C);
    e->g[OA_QA_CONV2_W] = ggml_new_tensor_4d(e->ctx, GGML_TYPE_F32, 3, 3, C, C);
    e->g[OA_QA_CONV3_W] = ggml_new_tensor_4d(e->ctx, GGML_TYPE_F32, 3, 3, C, C);
    for (int kind : {OA_QA_CONV1_B, OA_QA_CONV2_B, OA_QA_CONV3_B}) e->g[kind] = ggml_new_tensor_1d(e->ctx, GGML_TYPE_F32, C);
    e->g[OA_QA_CONV_OUT] = ggml_new_tensor_2d(e->ctx, wt, ck, d);
    for (int kind : {OA_QA_CONV_OUT_B, OA_QA_LN_POST_W, OA_QA_LN_POST_B, OA_QA_PROJ1_B})
        e->g[kind] = ggml_new_tensor_1d(e->ctx, GGML_TYPE_F32, d);
    e->g[OA_QA_PROJ1] = ggml_new_tensor_2d(e->ctx, wt, d, d);
    e->g[OA_QA_PROJ2] = ggml_new_tensor_2d(e->ctx, wt, d, c.out_dim);
    e->g[OA_QA_PROJ2_B] = ggml_new_tensor_1d(e->ctx, GGML_TYPE_F32, c.out_dim);
    e->g[OA_QA_INV_TIMESCALES] = ggml_new_tensor_2d(e->ctx, GGML_TYPE_F32, 1, d / 2);
    e->L.assign((size_t) c.n_layers, std::vector<ggml_tensor *>(OA_QA_LAYER_KINDS, nullptr));
    for (int l = 0; l < c.n_layers; l++) {
        for (int kind = 0; kind < OA_QA_LAYER_KINDS; kind++) {
            ggml_tensor *& t = e->L[(size_t) l][(size_t) kind];
            if (is_layer_matrix(kind)) {
                const int64_t rows = kind == OA_QA_UP ? c.ffn : d;
                const int64_t k = kind == OA_QA_DOWN ? c.ffn : d;
                t = ggml_new_tensor_2d(e->ctx, wt, k, rows);
            } else {
                t = ggml_new_tensor_1d(e->ctx, GGML_TYPE_F32, kind == OA_QA_UP_B ? c.ffn : d);
            }
        }
    }
    e->buf = ggml_backend_alloc_ctx_tensors_from_buft(e->ctx, ggml_backend_get_default_buffer_type(backend));
    if (!e->buf) {
        ggml_free(e->ctx);
        delete e;
        return nullptr;
    }
    ggml_backend_buffer_set_usage(e->buf, GGML_BACKEND_BUFFER_USAGE_WEIGHTS);
    for (auto & kv : e->g) {
        size_t n = 0;
        const void * src = oa_qwen_audio_weights_tensor(w, -1, kv.first, &n);
        if (src) ggml_backend_tensor_set(kv.second, src, 0, n);
    }
    for (int l = 0; l < c.n_layers; l++) {
        for (int kind = 0; kind < OA_QA_LAYER_KINDS; kind++) {
            size_t n = 0;
            const void * src = oa_qwen_audio_weights_tensor(w, l, kind, &n);
            ggml_backend_tensor_set(e->L[(size_t) l][(size_t) kind], src, 0, n);
        }
    }
    return e;
}

void oa_qwen_audio_encoder_free(oa_qwen_audio_encoder * e) {
    if (!e) return;
    e->release_graph();
    ggml_backend_buffer_free(e->buf);
    ggml_free(e->ctx);
    delete e;
}

int oa_qwen_audio_encoder_set_flash_attention_precision(oa_qwen_audio_encoder * e, int precision) {
    if (precision != GGML_PREC_DEFAULT && precision != GGML_PREC_F32) return GGML_STATUS_FAILED;
    if (precision != e->fa_prec) {
        e->fa_prec = precision;
        e->release_graph();
    }
    return GGML_STATUS_SUCCESS;
}

int oa_qwen_audio_encode(oa_qwen_audio_encoder * e, const float * mel, int n_frames, float * out, double * ms) {
    const oa_qwen_audio_config & c = e->cfg;
    if (n_frames <= 0 || !mel || !out) return GGML_STATUS_FAILED;
    const int chunks = (n_frames + kChunkFrames - 1) / kChunkFrames;
    const int cof = conv_out_len(conv_out_len(conv_out_len(kChunkFrames)));
    const int rows = chunks * cof;
    if (e->graph_chunks != chunks) {
        e->release_graph();
        if (!build_graph(e, chunks)) {
            e->release_graph();
            return GGML_STATUS_ALLOC_FAILED;
        }
    }
    // pack_mel_into_chunked_layout (:798-845): [chunk][mel][100 frames], the
    // tail chunk zero-padded
    std::vector<float> packed((size_t) chunks * c.n_mels * kChunkFrames, 0.0f);
    for (int ch = 0; ch < chunks; ch++) {
        const int f0 = ch * kChunkFrames, len = std::min(kChunkFrames, n_frames - f0);
        for (int m = 0; m < c.n_mels; m++)
            std::memcpy(&packed[((size_t) ch * c.n_mels + m) * kChunkFrames], mel + (size_t) m * n_frames + f0,
                        (size_t) len * sizeof(float));
    }
    std::vector<float> pos((size_t) cof);
    for (int i = 0; i < cof; i++) pos[(size_t) i] = (float) i;
    std::vector<float> mask((size_t) rows * rows, 0.0f);  // every row attends to every row (:341-345)
    ggml_backend_tensor_set(e->mel, packed.data(), 0, packed.size() * sizeof(float));
    ggml_backend_tensor_set(e->pos, pos.data(), 0, pos.size() * sizeof(float));
    ggml_backend_tensor_set(e->mask, mask.data(), 0, mask.size() * sizeof(float));
    const auto t0 = std::chrono::steady_clock::now();
    const int st = ggml_backend_graph_compute(e->backend, e->gf);
    if (st != GGML_STATUS_SUCCESS) return st;
    ggml_backend_tensor_get(e->out, out, 0, (size_t) rows * c.out_dim * sizeof(float));
    if (ms) *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return GGML_STATUS_SUCCESS;
}

}  // extern "C"

namespace {

std::vector<uint8_t> f32_bytes_of(const void * p, int type, int64_t n) {
    std::vector<float> v((size_t) n);
    if (type == GGML_TYPE_F32) std::memcpy(v.data(), p, (size_t) n * 4);
    else
        for (int64_t i = 0; i < n; i++) v[(size_t) i] = ggml_fp16_to_fp32(((const ggml_fp16_t *) p)[i]);
    return bytes_of(v);
}

}  // namespace

extern "C" {

// The names and checks of load_qwen3_audio_encoder_weights_from_reader
// (audio_encoder.rs:896-1050; names models/qwen/tensor_names.rs:3-45; keys
// arch/hparams.rs:42-52): float tensors (conv kernels, norms, biases) may be
// F32 or F16 and are widened to f32, as load_tensor_f32 does; the 2-D
// projections are bound in their stored type, one of F32 / F16 / Q8_0 for
// all of them.
oa_qwen_audio_weights * oa_qwen_audio_weights_load_gguf(const char * path, char * err, size_t err_cap) {
    auto report = [&](const std::string & msg) -> oa_qwen_audio_weights * {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", msg.c_str());
        return nullptr;
    };
    char gerr[256] = {0};
    oa_gguf * g = oa_gguf_open(path, gerr, sizeof(gerr));
    if (!g) return report(gerr);
    oa_pack::pack_reader r{g, {}};
    oa_qwen_audio_weights * w = new oa_qwen_audio_weights;
    auto bad = [&](const std::string & msg) {
        delete w;
        oa_gguf_close(g);
        return report(msg);
    };
    if (const char * a = oa_gguf_get_str(g, "general.architecture"); a && std::strcmp(a, "qwen3-asr") != 0)
        return bad(std::string("general.architecture is ") + a + ", not qwen3-asr");
    oa_qwen_audio_config & c = w->cfg;
    c = oa_qwen_audio_config{};
    if (!r.key_i("qwen3-asr.n_mels", c.n_mels) || !r.key_i("qwen3-asr.audio.n_layers", c.n_layers) ||
        !r.key_i("qwen3-asr.audio.d_model", c.d_model) || !r.key_i("qwen3-asr.audio.n_heads", c.n_heads) ||
        !r.key_i("qwen3-asr.llm.d_model", c.out_dim))
        return bad(r.err);
    if (c.d_model % c.n_heads != 0 || c.d_model % 2 != 0) return bad("audio.d_model is not an even multiple of audio.n_heads");
    w->freq_bins = conv_out_len(conv_out_len(conv_out_len(c.n_mels)));
    // rank-4 conv kernels [3, 3, IC, OC]
    auto conv = [&](const char * name, int64_t ic, int64_t oc, int kind) {
        const int64_t i = oa_gguf_find_tensor(g, name);
        if (i < 0) return r.fail(std::string("missing tensor ") + name);
        int type = 0;
        int64_t ne[4];
        oa_gguf_tensor_info(g, i, &type, ne);
        if (ne[0] != 3 || ne[1] != 3 || ne[2] != ic || (oc > 0 && ne[3] != oc))
            return r.fail(std::string("tensor ") + name + " is not a 3x3 kernel over the expected channels");
        if (type != GGML_TYPE_F32 && type != GGML_TYPE_F16) return r.fail(std::string("tensor ") + name + " is not F32 or F16");
        size_t nb = 0;
        w->global[kind] = f32_bytes_of(oa_gguf_tensor_data(g, i, &nb), type, 9 * ic * ne[3]);
        if (oc <= 0) c.conv_channels = (int) ne[3];
        return true;
    };
    auto vecf = [&](const std::string & name, int64_t n, std::vector<uint8_t> & out) {
        int type = 0;
        const int64_t i = r.tensor(name, n, 1, {GGML_TYPE_F32, GGML_TYPE_F16}, type);
        if (i < 0) return false;
        size_t nb = 0;
        out = f32_bytes_of(oa_gguf_tensor_data(g, i, &nb), type, n);
        return true;
    };
    int wtype = -1;
    auto mat = [&](const std::string & name, int64_t k, int64_t rows, std::vector<uint8_t> & out) {
        int type = 0;
        const int64_t i = r.tensor(name, k, rows, {GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_Q8_0}, type);
        if (i < 0) return false;
        if (wtype < 0) wtype = type;
        if (type != wtype)
            return r.fail("tensor " + name + " is " + ggml_type_name((ggml_type) type) + ", the encoder's projections are " +
                          ggml_type_name((ggml_type) wtype));
        size_t nb = 0;
        const uint8_t * p = (const uint8_t *) oa_gguf_tensor_data(g, i, &nb);
        out.assign(p, p + nb);
        return true;
    };
    if (!conv("audio.conv.1.weight", 1, 0, OA_QA_CONV1_W)) return bad(r.err);
    const int C = c.conv_channels, d = c.d_model;
    if (!conv("audio.conv.2.weight", C, C, OA_QA_CONV2_W) || !conv("audio.conv.3.weight", C, C, OA_QA_CONV3_W) ||
        !vecf("audio.conv.1.bias", C, w->global[OA_QA_CONV1_B]) || !vecf("audio.conv.2.bias", C, w->global[OA_QA_CONV2_B]) ||
        !vecf("audio.conv.3.bias", C, w->global[OA_QA_CONV3_B]) ||
        !mat("audio.conv_out.weight", (int64_t) C * w->freq_bins, d, w->global[OA_QA_CONV_OUT]) ||
        !vecf("audio.ln_post.weight", d, w->global[OA_QA_LN_POST_W]) ||
        !vecf("audio.ln_post.bias", d, w->global[OA_QA_LN_POST_B]) ||
        !mat("audio.proj1.weight", d, d, w->global[OA_QA_PROJ1]) || !vecf("audio.proj1.bias", d, w->global[OA_QA_PROJ1_B]) ||
        !mat("audio.proj2.weight", d, c.out_dim, w->global[OA_QA_PROJ2]) ||
        !vecf("audio.proj2.bias", c.out_dim, w->global[OA_QA_PROJ2_B]))
        return bad(r.err);
    w->conv_out_bias = oa_gguf_find_tensor(g, "audio.conv_out.bias") >= 0;
    if (w->conv_out_bias && !vecf("audio.conv_out.bias", d, w->global[OA_QA_CONV_OUT_B])) return bad(r.err);
    w->layers.assign((size_t) c.n_layers, std::vector<std::vector<uint8_t>>(OA_QA_LAYER_KINDS));
    for (int l = 0; l < c.n_layers; l++) {
        auto & L = w->layers[(size_t) l];
        const std::string p = "audio.blk." + std::to_string(l) + ".";
        // the FFN width comes from ffn_up's rows
        const int64_t up = oa_gguf_find_tensor(g, (p + "ffn_up.weight").c_str());
        if (up < 0) return bad("missing tensor " + p + "ffn_up.weight");
        int t = 0;
        int64_t ne[4];
        oa_gguf_tensor_info(g, up, &t, ne);
        if (l == 0) c.ffn = (int) ne[1];
        if (!vecf(p + "attn_norm.weight", d, L[OA_QA_ATTN_NORM_W]) || !vecf(p + "attn_norm.bias", d, L[OA_QA_ATTN_NORM_B]) ||
            !mat(p + "attn_q.weight", d, d, L[OA_QA_Q]) || !vecf(p + "attn_q.bias", d, L[OA_QA_Q_B]) ||
            !mat(p + "attn_k.weight", d, d, L[OA_QA_K]) || !vecf(p + "attn_k.bias", d, L[OA_QA_K_B]) ||
            !mat(p + "attn_v.weight", d, d, L[OA_QA_V]) || !vecf(p + "attn_v.bias", d, L[OA_QA_V_B]) ||
            !mat(p + "attn_out.weight", d, d, L[OA_QA_O]) || !vecf(p + "attn_out.bias", d, L[OA_QA_O_B]) ||
            !vecf(p + "ffn_norm.weight", d, L[OA_QA_FFN_NORM_W]) || !vecf(p + "ffn_norm.bias", d, L[OA_QA_FFN_NORM_B]) ||
            !mat(p + "ffn_up.weight", d, c.ffn, L[OA_QA_UP]) || !vecf(p + "ffn_up.bias", c.ffn, L[OA_QA_UP_B]) ||
            !mat(p + "ffn_down.weight", c.ffn, d, L[OA_QA_DOWN]) || !vecf(p + "ffn_down.bias", d, L[OA_QA_DOWN_B]))
            return bad(r.err);
    }
    c.wtype = wtype;
    if (c.wtype == GGML_TYPE_Q8_0 && (((int64_t) C * w->freq_bins) % 32 || d % 32 || c.ffn % 32))
        return bad("Q8_0 projections need every K % 32 == 0");
    const int half = d / 2;
    const float log_inc = std::log(10000.0f) / (float) (half - 1 > 1 ? half - 1 : 1);
    std::vector<float> inv((size_t) half);
    for (int i = 0; i < half; i++) inv[(size_t) i] = std::exp(-log_inc * (float) i);
    w->global[OA_QA_INV_TIMESCALES] = bytes_of(inv);
    oa_gguf_close(g);
    return w;
}

void oa_qwen_audio_weights_config(const oa_qwen_audio_weights * w, oa_qwen_audio_config * out) { *out = w->cfg; }

}  // extern "C"
