/*
 * openasr_models.h -- the decoder families on the quantized decoder path, as
 * the OpenASR host drives them through ggml (libopenasr-models.so). These are
 * the host-side callers of the backend plugin: they build the same ggml graphs
 * the Rust emitters build and run the same greedy step loops.
 *
 * Qwen3 LLM decoder: compose_llm_decoder_layer_stack / llm_layer
 *   (crates/openasr-core/src/nn/decoder.rs:1850-2331), persistent reusable
 *   decode graph with a resident f16 KV arena and per-step token / row /
 *   position / mask uploads (models/qwen/llm_transformer.rs:5169-5657),
 *   fused logits head with first-max top-1 (llm_transformer.rs:2096-2115),
 *   prefill in chunks of at most 256 query tokens (llm_transformer.rs:60,
 *   4016-4200).
 * Greedy n-gram loop guard: models/seq2seq_greedy_decode.rs:19-58, 569-605.
 *
 * Weights are synthesised (seeded N(0, 0.02), then quantized with
 * ggml_quantize_chunk); the host copy stays available so a CPU checker can
 * consume exactly the bytes the device holds.
 */
#ifndef OPENASR_MODELS_H
#define OPENASR_MODELS_H

#include "ggml_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int d_model;
    int n_layers;
    int n_head;
    int n_kv_head;
    int head_dim;
    int ffn;
    int vocab;
    float rope_theta;
    float rms_eps;
    int wtype; /* GGML_TYPE_Q8_0 or GGML_TYPE_Q4_K for every matrix and the tied embedding */
    uint64_t seed;
    int out_wtype; /* type of a separate output projection (runtime packs with output.weight), else unused */
} oa_qwen_config;

enum oa_qwen_tensor_kind {
    OA_QWEN_TOKEN_EMBD = 0, /* [vocab rows of d_model], wtype; tied with the lm_head */
    OA_QWEN_OUTPUT_NORM,    /* f32 [d_model] */
    OA_QWEN_ATTN_NORM,      /* f32 [d_model] */
    OA_QWEN_QKV,            /* wtype, rows q|k|v of d_model: the fused projection */
    OA_QWEN_Q_NORM,         /* f32 [head_dim] */
    OA_QWEN_K_NORM,         /* f32 [head_dim] */
    OA_QWEN_O,              /* wtype, d_model rows of n_head*head_dim */
    OA_QWEN_FFN_NORM,       /* f32 [d_model] */
    OA_QWEN_GATE,           /* wtype, ffn rows of d_model */
    OA_QWEN_UP,             /* wtype, ffn rows of d_model */
    OA_QWEN_DOWN,           /* wtype, d_model rows of ffn */
    OA_QWEN_OUTPUT          /* out_wtype [vocab rows of d_model]: a separate output projection, NULL when tied */
};

typedef struct oa_qwen_weights oa_qwen_weights;

/*
 * GGUF runtime-pack reader (v2/v3, the `.oasr` v1 payload:
 * docs/format/OASR_PACKAGE_CONTRACT_V1.md). The file is mapped read-only;
 * tensor data are views into the mapping, valid until oa_gguf_close. The
 * reserved OASR magic and unknown magics are refused, as are malformed
 * headers, out-of-file or misaligned tensor ranges and duplicate names
 * (the fork's gguf_init_from_file + ggml_runtime/gguf_tensor_data.rs).
 */
typedef struct oa_gguf oa_gguf;
oa_gguf * oa_gguf_open(const char * path, char * err, size_t err_cap);
void oa_gguf_close(oa_gguf * g);
uint32_t oa_gguf_version(const oa_gguf * g);
size_t oa_gguf_alignment(const oa_gguf * g);
int64_t oa_gguf_n_tensors(const oa_gguf * g);
int64_t oa_gguf_n_kv(const oa_gguf * g);
int64_t oa_gguf_find_tensor(const oa_gguf * g, const char * name); /* -1 when absent */
const char * oa_gguf_tensor_name(const oa_gguf * g, int64_t i);
/* type and ne[4] of tensor i; returns n_dims, -1 for a bad index */
int oa_gguf_tensor_info(const oa_gguf * g, int64_t i, int * type, int64_t ne[4]);
const void * oa_gguf_tensor_data(const oa_gguf * g, int64_t i, size_t * nbytes);
int oa_gguf_kv_type(const oa_gguf * g, const char * key); /* GGUF value type, -1 when absent */
const char * oa_gguf_get_str(const oa_gguf * g, const char * key);
bool oa_gguf_get_i64(const oa_gguf * g, const char * key, int64_t * out);  /* any integer type */
bool oa_gguf_get_f64(const oa_gguf * g, const char * key, double * out);   /* float or integer */
typedef struct oa_qwen_model oa_qwen_model;
typedef struct oa_qwen_session oa_qwen_session;

oa_qwen_weights * oa_qwen_weights_synthesize(const oa_qwen_config * cfg);
/* Weights of a qwen3-asr runtime pack (.oasr v1 = GGUF): hparams from the
 * qwen3-asr.llm.* keys (arch/hparams.rs:52-58), tensors blk.N.{attn_norm,
 * attn_q, attn_k, attn_v, attn_output, attn_q_norm, attn_k_norm, ffn_norm,
 * ffn_gate, ffn_up, ffn_down}.weight, token_embd.weight, output_norm.weight
 * and an optional output.weight (models/qwen/decoder_contract.rs:686-705,
 * 764-769). The matrices stay views into the file mapping (q|k|v are joined
 * into the fused projection, llm_transformer.rs:6505-6555); every matrix must
 * be Q8_0 or Q4_K, all of one type. RoPE theta 1e6 unless the pack carries
 * qwen3-asr.llm.rope_theta; RMS epsilon 1e-6. NULL with a message on any
 * missing or mis-shaped tensor or key. */
oa_qwen_weights * oa_qwen_weights_load_gguf(const char * path, char * err, size_t err_cap);
/* the configuration the weights describe */
void oa_qwen_weights_config(const oa_qwen_weights * w, oa_qwen_config * out);
void oa_qwen_weights_free(oa_qwen_weights * w);
/* host bytes of one tensor (layer ignored for TOKEN_EMBD / OUTPUT_NORM) */
const void * oa_qwen_weights_tensor(const oa_qwen_weights * w, int layer, int kind, size_t * nbytes);

oa_qwen_model * oa_qwen_model_create(ggml_backend_t backend, const oa_qwen_weights * w);
void oa_qwen_model_free(oa_qwen_model * m);

oa_qwen_session * oa_qwen_session_create(oa_qwen_model * m, int n_seq, int max_positions);
void oa_qwen_session_free(oa_qwen_session * s);
int oa_qwen_session_position(const oa_qwen_session * s, int seq);

/* Greedy top-1 head of the session's step graphs: 0 (default) ARGMAX_FIRST
 * over the logits; 1 the reversed-row graph of the whole-decoder fused
 * logits head (cpu_graph.rs:3772-3810, llm_transformer.rs:2096-2130) --
 * GET_ROWS by vocab - 1 .. 0 (through a transposed copy for more than one
 * sequence), CONT, then ggml's last-max ARGMAX, the result r mapped to
 * vocab - 1 - r; a result outside the vocabulary fails the step. Both give
 * the first of equal maxima. Takes effect on the next step. */
void oa_qwen_session_set_reversed_top1(oa_qwen_session * s, int enable);

/* The step graphs the unmodified host builds on a discrete-GPU HIP backend
 * (enable = 1): native GQA is Unsupported there
 * (ggml_runtime/cpu_graph.rs:736-757), so each layer expands K and V to the
 * query heads with RESHAPE / REPEAT / RESHAPE (expand_attention_kv,
 * nn/decoder.rs:1799-1841); prefill chunks of more than two positions over
 * a span of more than 32 take the unfused attention chain
 * (llm_naive_masked_attention, nn/decoder.rs:2154-2200;
 * llm_transformer.rs:7864-7877) with GGML_PREC_F32 on its two products
 * (cpu_graph.rs:157-165, 202-228); prefill runs in chunks of at most
 * prefill_chunk positions, odd widths above one trimmed by one
 * (llm_transformer.rs:7903-7911). One sequence only, as the host refuses
 * more on this lane (llm_transformer.rs:2444-2450): another n_seq returns
 * GGML_STATUS_FAILED. Takes effect on the next step. */
int oa_qwen_session_set_hip_lane(oa_qwen_session * s, int enable, int prefill_chunk);

/* The precision contract of the self-attention's FLASH_ATTN_EXT
 * (set_flash_attention_precision, models/qwen/llm_transformer.rs:3044-3053;
 * GgmlFlashAttentionPrecision, ggml_runtime/cpu_graph.rs:122-155):
 * GGML_PREC_DEFAULT (the default, what the ASR decoder builds) lets the
 * backend take its fastest validated form within float tolerance -- prefill
 * chunks on the matrix cores, decode steps one workgroup per (sequence, kv
 * head) with the combine in the launch; GGML_PREC_F32 (what the forced
 * aligner selects, forced_aligner_runtime.rs:622) keeps every attention in
 * the exact chunked form. Other values return GGML_STATUS_FAILED. Takes
 * effect on the next step. */
int oa_qwen_session_set_flash_attention_precision(oa_qwen_session * s, int precision);

/* The precision of the quantized projections' MUL_MATs (GgmlMatmulPrecision,
 * ggml_runtime/cpu_graph.rs:142-146; mul_mat / mul_mat_impl :3615-3685 set
 * GGML_PREC_F32 only on request, and the decoder's projections,
 * nn/decoder.rs:1621, take the plain mul_mat): GGML_PREC_DEFAULT (the
 * default) lets wide prefill products run on the f16 matrix cores within
 * float tolerance; GGML_PREC_F32 keeps every product in the exact integer
 * form. Decode-size products are exact under both. Other values return
 * GGML_STATUS_FAILED. Takes effect on the next step. */
int oa_qwen_session_set_matmul_precision(oa_qwen_session * s, int precision);

/* Prefill T positions of every sequence (chunked internally at 256) from
 * hidden inputs [n_seq][T][d_model] (an audio-embedding prefix) or token ids
 * [n_seq][T]. top1_out (optional, [n_seq]) gets the first-max argmax of the
 * last position's logits. Returns a ggml_status. */
int oa_qwen_prefill_embeddings(oa_qwen_session * s, const float * emb, int T, int32_t * top1_out);
int oa_qwen_prefill_tokens(oa_qwen_session * s, const int32_t * tokens, int T, int32_t * top1_out);

/* One decode step for every sequence: tokens [n_seq] in, top-1 [n_seq] out
 * (lowest index on ties). logits_out (optional) gets [n_seq][vocab]. */
int oa_qwen_decode_step(oa_qwen_session * s, const int32_t * tokens, int32_t * top1_out, float * logits_out);

/* Greedy loop: feeds each step's top-1 back in for n_steps steps.
 * out_tokens [n_steps][n_seq]; step_ms (optional) wall time per step. */
int oa_qwen_generate(oa_qwen_session * s, const int32_t * first_tokens, int n_steps, int32_t * out_tokens,
                     double * step_ms);

/* Device KV cache of one layer for one sequence, f16 bits [n_kv_head][max_positions][head_dim] each. */
int oa_qwen_read_kv(const oa_qwen_session * s, int layer, int seq, uint16_t * k_out, uint16_t * v_out);

/* The persistent decode-step graph (built on the first decode step; NULL
 * before), for measurement hooks that replay it. */
struct ggml_cgraph * oa_qwen_decode_graph(oa_qwen_session * s);

/* Degenerate n-gram guard (seq2seq_greedy_decode.rs:569-605): smallest n in
 * 1..max_ngram whose trailing n-gram repeats at least bounds[n - 1] times
 * back to back (the reference's max_consecutive_repeats(n) function as a
 * table; a bound of 0 disables that length). bounds == NULL selects the
 * shipped tiers, default_max_consecutive_ngram_repeats (:51-58): 8 for n=1,
 * 6 for n=2, 4 for n>=3. Returns the length to keep (the run truncated to one
 * occurrence: len - (repeats - 1) * n), or -1 when no loop is detected (also
 * for max_ngram 0 or an empty tail). */
int oa_detect_degenerate_ngram(const int32_t * tokens, int len, int max_ngram, const int * bounds, int * ngram_len,
                               int * repeats);

/*
 * Whisper decoder (models/whisper/ggml_decoder_graph.rs): reusable one-token
 * step graph (:3869-4052) -- token + learned position embedding, per layer
 * pre-LayerNorm self attention over a resident f16 KV cache with the
 * fixed-span mask (:4557-5044), cross attention over the precomputed f16
 * cross K/V of the encoder frames (:5106-5340), LayerNorm -> fc1 -> GELU ->
 * fc2 MLP (:5342-5392), each with its residual; final LayerNorm and the
 * output projection tied to the token embedding. Cross K/V are precomputed
 * once per utterance: K = Wk enc, V = Wv enc + bv, stored f16 (:5780-5805).
 * Batch 1.
 */
typedef struct {
    int d_model;
    int n_layers;
    int n_head;
    int ffn;
    int vocab;
    int max_positions; /* learned positions and the self KV span */
    int n_frames;      /* encoder frames the cross attention reads */
    float ln_eps;
    uint64_t seed;
    /* FFN activation between fc1 and fc2 of the shared seq2seq block
     * (nn/decoder.rs:1125-1138): 0 GELU (Whisper), 1 RELU, 2 GELU_ERF, 3 SILU */
    int ffn_act;
} oa_whisper_config;

enum oa_whisper_tensor_kind {
    /* per layer (layer >= 0); matrices Q8_0 rows of d_model (fc2: rows of ffn), vectors f32 */
    OA_WH_SELF_LN_W = 0, OA_WH_SELF_LN_B, OA_WH_SELF_Q, OA_WH_SELF_Q_B, OA_WH_SELF_K, OA_WH_SELF_V,
    OA_WH_SELF_V_B, OA_WH_SELF_O, OA_WH_SELF_O_B,
    OA_WH_CROSS_LN_W, OA_WH_CROSS_LN_B, OA_WH_CROSS_Q, OA_WH_CROSS_Q_B, OA_WH_CROSS_K, OA_WH_CROSS_V,
    OA_WH_CROSS_V_B, OA_WH_CROSS_O, OA_WH_CROSS_O_B,
    OA_WH_MLP_LN_W, OA_WH_MLP_LN_B, OA_WH_FC1, OA_WH_FC1_B, OA_WH_FC2, OA_WH_FC2_B,
    OA_WH_LAYER_KINDS,
    /* global (layer = -1) */
    OA_WH_TOKEN_EMBD = 100, /* Q8_0 [vocab rows of d_model], tied with the output projection */
    OA_WH_POS_EMBD,         /* f32 [max_positions rows of d_model] */
    OA_WH_FINAL_LN_W,
    OA_WH_FINAL_LN_B
};

typedef struct oa_whisper_weights oa_whisper_weights;
typedef struct oa_whisper_model oa_whisper_model;
typedef struct oa_whisper_session oa_whisper_session;

oa_whisper_weights * oa_whisper_weights_synthesize(const oa_whisper_config * cfg);
void oa_whisper_weights_free(oa_whisper_weights * w);
const void * oa_whisper_weights_tensor(const oa_whisper_weights * w, int layer, int kind, size_t * nbytes);

/* A whisper runtime pack (.oasr v1, GGUF v2/v3): hparams whisper.decoder.{block_count,
 * embedding_length, attention.head_count, context_length}, whisper.vocab_size and
 * whisper.encoder.context_length (models/whisper/runtime_contract.rs:180-230);
 * decoder tensors decoder.token_embedding.weight (Q8_0, tied output projection),
 * decoder.positional_embedding (F32), decoder.layer_norm.{weight,bias} and per layer
 * decoder.layers.N.{self_attn,cross_attn}.{q,k,v,out}_proj.* (k without bias),
 * {self_attn,encoder_attn,final}_layer_norm.*, fc1.*, fc2.* (ggml_tensor_binding.rs:135-210),
 * matrices Q8_0. Matrices stay views into the read-only mapping (released with
 * the weights). NULL and a message in err on any missing key or tensor, wrong
 * shape or type. */
oa_whisper_weights * oa_whisper_weights_load_gguf(const char * path, char * err, size_t err_cap);
void oa_whisper_weights_config(const oa_whisper_weights * w, oa_whisper_config * out);

oa_whisper_model * oa_whisper_model_create(ggml_backend_t backend, const oa_whisper_weights * w);
void oa_whisper_model_free(oa_whisper_model * m);

oa_whisper_session * oa_whisper_session_create(oa_whisper_model * m);
void oa_whisper_session_free(oa_whisper_session * s);
int oa_whisper_session_position(const oa_whisper_session * s);
/* encoder states [n_frames][d_model] f32 -> the per-layer f16 cross K/V */
int oa_whisper_set_encoder(oa_whisper_session * s, const float * enc);
/* one token at the next position; top-1 (first max) and optionally the logits */
int oa_whisper_decode_step(oa_whisper_session * s, int32_t token, int32_t * top1_out, float * logits_out);
int oa_whisper_generate(oa_whisper_session * s, int32_t first_token, int n_steps, int32_t * out_tokens,
                        double * step_ms);
/* the layer's cross K / V caches, f16 [n_frames][d_model] */
int oa_whisper_read_cross(const oa_whisper_session * s, int layer, uint16_t * k_out, uint16_t * v_out);
/* the layer's self-attention K / V caches, f16 [max_positions][d_model] (row
 * p written by the step at position p) */
int oa_whisper_read_self(const oa_whisper_session * s, int layer, uint16_t * k_out, uint16_t * v_out);
/* The precision contract of the decoder's self and cross FLASH_ATTN_EXT
 * (flash_attention_precision of the seq2seq decoder graphs, nn/decoder.rs:
 * 3064-3728): GGML_PREC_DEFAULT (the default) runs the single-query
 * workgroup form within float tolerance, GGML_PREC_F32 the exact chunked
 * form. Other values return GGML_STATUS_FAILED. Takes effect on the next
 * step. */
int oa_whisper_session_set_flash_attention_precision(oa_whisper_session * s, int precision);
struct ggml_cgraph * oa_whisper_decode_graph(oa_whisper_session * s);

/* ---- Qwen3-ASR audio encoder (crates/openasr-core/src/models/qwen/audio_encoder.rs) ----
 * The prefix producer of the Qwen decoder, as the host builds its graph for a
 * GPU backend (flash attention over strided head views): mel [n_mels][n_frames]
 * packed into 100-frame chunks (:798-845), three 3x3 stride-2 GELU_ERF
 * convolutions with f32 kernels (:510-552, nn/conv.rs:82-111), the channel
 * permute and conv_out projection (:553-592), the sinusoidal position table
 * added per chunk (:455-465, nn/encoder.rs:575-590), n_layers pre-norm
 * encoder blocks over all chunks' rows with a zero f32 mask cast to f16
 * (:1078-1110, nn/encoder.rs:678-870), ln_post, proj1 + GELU_ERF, proj2
 * (:615-672). Output: [rows][out_dim] f32, rows = 13 per chunk
 * (qwen3_audio_token_count_for_mel_frames, :859-867). */
typedef struct oa_qwen_audio_config {
    int n_mels;         /* mel bins (even, >= 8) */
    int conv_channels;  /* channels of the three convolutions */
    int d_model, n_heads, n_layers, ffn;
    int out_dim;        /* the decoder's d_model */
    int wtype;          /* 2-D projections: GGML_TYPE_F32, GGML_TYPE_F16 or GGML_TYPE_Q8_0 */
    uint64_t seed;
} oa_qwen_audio_config;

enum oa_qwen_audio_tensor_kind {
    /* per layer (layer >= 0); matrices [rows][K] of wtype, vectors f32 */
    OA_QA_ATTN_NORM_W = 0, OA_QA_ATTN_NORM_B, OA_QA_Q, OA_QA_Q_B, OA_QA_K, OA_QA_K_B, OA_QA_V, OA_QA_V_B,
    OA_QA_O, OA_QA_O_B, OA_QA_FFN_NORM_W, OA_QA_FFN_NORM_B, OA_QA_UP, OA_QA_UP_B, OA_QA_DOWN, OA_QA_DOWN_B,
    OA_QA_LAYER_KINDS,
    /* global (layer = -1): f32 conv kernels [OC][IC][3][3] (ggml [3, 3, IC, OC]) and biases */
    OA_QA_CONV1_W = 100, OA_QA_CONV1_B, OA_QA_CONV2_W, OA_QA_CONV2_B, OA_QA_CONV3_W, OA_QA_CONV3_B,
    OA_QA_CONV_OUT, OA_QA_CONV_OUT_B, /* matrix [d_model][conv_channels * freq bins] of wtype */
    OA_QA_LN_POST_W, OA_QA_LN_POST_B,
    OA_QA_PROJ1, OA_QA_PROJ1_B, /* [d_model][d_model] */
    OA_QA_PROJ2, OA_QA_PROJ2_B, /* [out_dim][d_model] */
    OA_QA_INV_TIMESCALES        /* f32 [d_model / 2]: exp(-ln(10000) i / (d_model / 2 - 1)) */
};

typedef struct oa_qwen_audio_weights oa_qwen_audio_weights;
typedef struct oa_qwen_audio_encoder oa_qwen_audio_encoder;

/* seeded N(0, 0.02) matrices quantized / rounded to wtype; NULL on a shape the
 * type cannot hold (Q8_0 needs every K % 32 == 0) */
oa_qwen_audio_weights * oa_qwen_audio_weights_synthesize(const oa_qwen_audio_config * cfg);
void oa_qwen_audio_weights_free(oa_qwen_audio_weights * w);
const void * oa_qwen_audio_weights_tensor(const oa_qwen_audio_weights * w, int layer, int kind, size_t * nbytes);
/* The encoder of a qwen3-asr runtime pack: keys qwen3-asr.n_mels,
 * qwen3-asr.audio.{n_layers,d_model,n_heads}, qwen3-asr.llm.d_model (arch/hparams.rs:42-52);
 * tensors audio.conv.{1,2,3}.{weight,bias}, audio.conv_out.weight (+ optional bias),
 * audio.ln_post.*, audio.proj{1,2}.*, audio.blk.N.{attn_norm,attn_q,attn_k,attn_v,
 * attn_out,ffn_norm,ffn_up,ffn_down}.{weight,bias} (models/qwen/tensor_names.rs:3-45);
 * conv kernels, norms and biases F32 or F16 (widened to f32), projections all
 * F32, F16 or Q8_0. The bytes are copied; the pack is closed on return. NULL
 * and a message in err on a missing key or tensor, a wrong shape or type. */
oa_qwen_audio_weights * oa_qwen_audio_weights_load_gguf(const char * path, char * err, size_t err_cap);
void oa_qwen_audio_weights_config(const oa_qwen_audio_weights * w, oa_qwen_audio_config * out);
/* rows the encoder emits for n_frames mel frames: 13 per started 100-frame chunk */
int oa_qwen_audio_token_count(int n_frames);
oa_qwen_audio_encoder * oa_qwen_audio_encoder_create(ggml_backend_t backend, const oa_qwen_audio_weights * w);
void oa_qwen_audio_encoder_free(oa_qwen_audio_encoder * e);
/* one encode: mel [n_mels][n_frames] f32 -> out [rows][out_dim] f32; ms (may be
 * NULL) receives the compute's wall time. The graph is built on the first call
 * for a chunk count and replayed after. Returns a ggml_status. */
int oa_qwen_audio_encode(oa_qwen_audio_encoder * e, const float * mel, int n_frames, float * out, double * ms);
/* The self-attention's FLASH_ATTN_EXT precision. The reference's encoder
 * always builds GGML_PREC_DEFAULT (flash_attn_ext, cpu_graph.rs:4120-4142;
 * nn/encoder.rs:784-793), this shim's default too: the matrix-core form
 * within float tolerance. GGML_PREC_F32 keeps the exact chunked form; this
 * switch has no counterpart in the reference and is there for exact
 * comparisons. Other values return GGML_STATUS_FAILED; the next encode
 * rebuilds the graph. */
int oa_qwen_audio_encoder_set_flash_attention_precision(oa_qwen_audio_encoder * e, int precision);

/* ---- pack storage policy (crates/openasr-core/src/models/pack_quant.rs) ---- */

/* requested pack rung, enum PackQuant (pack_quant.rs:25-32) */
enum oa_pack_quant { OA_PACK_FP16 = 0, OA_PACK_Q8_0 = 1, OA_PACK_Q3_K = 2, OA_PACK_Q4_K = 3 };
/* a tensor's mathematical role, enum TensorRole (pack_quant.rs:51-62) */
enum oa_tensor_role {
    OA_ROLE_ACOUSTIC_ENCODER_MATRIX = 0,
    OA_ROLE_TEXT_DECODER_MATRIX = 1,
    OA_ROLE_EMBEDDING_TABLE = 2,
    OA_ROLE_OUTPUT_PROJECTION = 3,
    OA_ROLE_PRECISION_CRITICAL_MATRIX = 4,
    OA_ROLE_NON_QUANTIZABLE = 5,
};
/* which dimension is ggml's ne0, enum QuantizedAxis (pack_quant.rs:64-68) */
enum oa_quantized_axis { OA_AXIS_FIRST = 0, OA_AXIS_LAST = 1 };

/* classify_quant_tensor_role (pack_quant.rs:179-213): the ggml type the
 * writer stores the tensor as (GGML_TYPE_Q8_0 / Q3_K / Q4_K), -1 for "keep
 * the rung's non-quantized representation" (the reference's None), -2 for
 * an argument out of range. */
int oa_classify_quant_tensor_role(const uint64_t * dims, int n_dims, int quantization, int role, int axis);
/* TensorQuantizationContract::target_write_type (pack_quant.rs:127-147) for
 * a resolved role and axis: only rank-2 tensors are block-quantized. Same
 * returns. */
int oa_quant_target_write_type(const uint64_t * dims, int n_dims, int quantization, int role, int axis);

#ifdef __cplusplus
}
#endif

#endif
