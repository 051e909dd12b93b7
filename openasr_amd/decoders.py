"""ctypes view of libopenasr-models.so (include/openasr_models.h): the decoder
families' graph builders and greedy step loops, driving the backend through
the ggml C ABI. Also the workload configurations the path is measured on.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import ggml as g

MODELS_PATH = g.LIB_DIR / "libopenasr-models.so"


class QwenConfig(C.Structure):
    _fields_ = [("d_model", C.c_int), ("n_layers", C.c_int), ("n_head", C.c_int), ("n_kv_head", C.c_int),
                ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("rope_theta", C.c_float),
                ("rms_eps", C.c_float), ("wtype", C.c_int), ("seed", C.c_uint64), ("out_wtype", C.c_int)]


class WhisperConfig(C.Structure):
    _fields_ = [("d_model", C.c_int), ("n_layers", C.c_int), ("n_head", C.c_int), ("ffn", C.c_int),
                ("vocab", C.c_int), ("max_positions", C.c_int), ("n_frames", C.c_int), ("ln_eps", C.c_float),
                ("seed", C.c_uint64), ("ffn_act", C.c_int)]


class QwenAudioConfig(C.Structure):
    _fields_ = [("n_mels", C.c_int), ("conv_channels", C.c_int), ("d_model", C.c_int), ("n_heads", C.c_int),
                ("n_layers", C.c_int), ("ffn", C.c_int), ("out_dim", C.c_int), ("wtype", C.c_int),
                ("seed", C.c_uint64)]


# Qwen3-ASR audio encoder tensor kinds (enum oa_qwen_audio_tensor_kind)
(QA_ATTN_NORM_W, QA_ATTN_NORM_B, QA_Q, QA_Q_B, QA_K, QA_K_B, QA_V, QA_V_B, QA_O, QA_O_B, QA_FFN_NORM_W,
 QA_FFN_NORM_B, QA_UP, QA_UP_B, QA_DOWN, QA_DOWN_B) = range(16)
QA_LAYER_KINDS = 16
(QA_CONV1_W, QA_CONV1_B, QA_CONV2_W, QA_CONV2_B, QA_CONV3_W, QA_CONV3_B, QA_CONV_OUT, QA_CONV_OUT_B,
 QA_LN_POST_W, QA_LN_POST_B, QA_PROJ1, QA_PROJ1_B, QA_PROJ2, QA_PROJ2_B, QA_INV_TIMESCALES) = range(100, 115)
# an audio encoder of Qwen3-ASR-0.6B's shape: 128 mel bins, 480 conv channels,
# 18 layers of d_model 896 (14 heads, FFN 3584), into a 1024-wide decoder
QWEN3_06B_AUDIO = dict(n_mels=128, conv_channels=480, d_model=896, n_heads=14, n_layers=18, ffn=3584, out_dim=1024)


# FFN activations of the shared seq2seq block (oa_whisper_config.ffn_act)
FFN_GELU, FFN_RELU, FFN_GELU_ERF, FFN_SILU = 0, 1, 2, 3


# Whisper-tiny decoder shape: d_model 384, 4 layers, 6 heads of 64, FFN 1536, vocab 51865,
# 448 learned positions, 1500 encoder frames
WHISPER_TINY = dict(d_model=384, n_layers=4, n_head=6, ffn=1536, vocab=51865, max_positions=448, n_frames=1500)
WH_LAYER_KINDS = 24
# per-layer tensor kinds (oa_whisper_tensor_kind)
(WH_SELF_LN_W, WH_SELF_LN_B, WH_SELF_Q, WH_SELF_Q_B, WH_SELF_K, WH_SELF_V, WH_SELF_V_B, WH_SELF_O, WH_SELF_O_B,
 WH_CROSS_LN_W, WH_CROSS_LN_B, WH_CROSS_Q, WH_CROSS_Q_B, WH_CROSS_K, WH_CROSS_V, WH_CROSS_V_B, WH_CROSS_O,
 WH_CROSS_O_B, WH_MLP_LN_W, WH_MLP_LN_B, WH_FC1, WH_FC1_B, WH_FC2, WH_FC2_B) = range(WH_LAYER_KINDS)
WH_TOKEN_EMBD, WH_POS_EMBD, WH_FINAL_LN_W, WH_FINAL_LN_B = 100, 101, 102, 103

# Qwen3-0.6B / 1.7B shapes (hidden, layers, heads, kv heads, head_dim, ffn, vocab)
QWEN3_06B = dict(d_model=1024, n_layers=28, n_head=16, n_kv_head=8, head_dim=128, ffn=3072, vocab=151936)
QWEN3_17B = dict(d_model=2048, n_layers=28, n_head=16, n_kv_head=8, head_dim=128, ffn=6144, vocab=151936)

# tensor kinds (enum oa_qwen_tensor_kind)
(TOKEN_EMBD, OUTPUT_NORM, ATTN_NORM, QKV, Q_NORM, K_NORM, O, FFN_NORM, GATE, UP, DOWN, OUTPUT) = range(12)
LAYER_KINDS = (ATTN_NORM, QKV, Q_NORM, K_NORM, O, FFN_NORM, GATE, UP, DOWN)

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    g.base()
    if not MODELS_PATH.exists():
        raise RuntimeError(f"{MODELS_PATH} is missing: run `python -m openasr_amd.build` first")
    L = C.CDLL(str(MODELS_PATH))
    vp, i, i32p = C.c_void_p, C.c_int, C.POINTER(C.c_int32)

    def s(name, res, *args):
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = list(args)

    s("oa_qwen_weights_synthesize", vp, C.POINTER(QwenConfig))
    s("oa_qwen_weights_load_gguf", vp, C.c_char_p, C.c_char_p, C.c_size_t)
    s("oa_qwen_weights_config", None, vp, C.POINTER(QwenConfig))
    i64 = C.c_int64
    s("oa_gguf_open", vp, C.c_char_p, C.c_char_p, C.c_size_t)
    s("oa_gguf_close", None, vp)
    s("oa_gguf_version", C.c_uint32, vp)
    s("oa_gguf_alignment", C.c_size_t, vp)
    s("oa_gguf_n_tensors", i64, vp)
    s("oa_gguf_n_kv", i64, vp)
    s("oa_gguf_find_tensor", i64, vp, C.c_char_p)
    s("oa_gguf_tensor_name", C.c_char_p, vp, i64)
    s("oa_gguf_tensor_info", i, vp, i64, C.POINTER(C.c_int), C.POINTER(i64))
    s("oa_gguf_tensor_data", vp, vp, i64, C.POINTER(C.c_size_t))
    s("oa_gguf_kv_type", i, vp, C.c_char_p)
    s("oa_gguf_get_str", C.c_char_p, vp, C.c_char_p)
    s("oa_gguf_get_i64", C.c_bool, vp, C.c_char_p, C.POINTER(i64))
    s("oa_gguf_get_f64", C.c_bool, vp, C.c_char_p, C.POINTER(C.c_double))
    s("oa_qwen_weights_free", None, vp)
    s("oa_qwen_weights_tensor", vp, vp, i, i, C.POINTER(C.c_size_t))
    s("oa_qwen_model_create", vp, vp, vp)
    s("oa_qwen_model_free", None, vp)
    s("oa_qwen_session_create", vp, vp, i, i)
    s("oa_qwen_session_free", None, vp)
    s("oa_qwen_session_position", i, vp, i)
    s("oa_qwen_session_set_reversed_top1", None, vp, i)
    s("oa_qwen_session_set_flash_attention_precision", i, vp, i)
    s("oa_qwen_session_set_matmul_precision", i, vp, i)
    s("oa_qwen_session_set_hip_lane", i, vp, i, i)
    s("oa_qwen_prefill_embeddings", i, vp, vp, i, vp)
    s("oa_qwen_prefill_tokens", i, vp, vp, i, vp)
    s("oa_qwen_decode_step", i, vp, vp, vp, vp)
    s("oa_whisper_weights_synthesize", vp, C.POINTER(WhisperConfig))
    s("oa_whisper_weights_free", None, vp)
    s("oa_whisper_weights_tensor", vp, vp, i, i, C.POINTER(C.c_size_t))
    s("oa_whisper_weights_load_gguf", vp, C.c_char_p, C.c_char_p, C.c_size_t)
    s("oa_whisper_weights_config", None, vp, C.POINTER(WhisperConfig))
    s("oa_whisper_model_create", vp, vp, vp)
    s("oa_whisper_model_free", None, vp)
    s("oa_whisper_session_create", vp, vp)
    s("oa_whisper_session_free", None, vp)
    s("oa_whisper_session_position", i, vp)
    s("oa_whisper_set_encoder", i, vp, vp)
    s("oa_whisper_decode_step", i, vp, C.c_int32, vp, vp)
    s("oa_whisper_generate", i, vp, C.c_int32, i, vp, vp)
    s("oa_whisper_read_cross", i, vp, i, vp, vp)
    s("oa_whisper_read_self", i, vp, i, vp, vp)
    s("oa_whisper_decode_graph", vp, vp)
    s("oa_whisper_session_set_flash_attention_precision", i, vp, i)
    s("oa_qwen_generate", i, vp, vp, i, vp, vp)
    s("oa_qwen_read_kv", i, vp, i, i, vp, vp)
    s("oa_detect_degenerate_ngram", i, vp, i, i, vp, vp, vp)
    s("oa_qwen_audio_weights_synthesize", vp, vp)
    s("oa_qwen_audio_weights_free", None, vp)
    s("oa_qwen_audio_weights_tensor", vp, vp, i, i, C.POINTER(C.c_size_t))
    s("oa_qwen_audio_token_count", i, i)
    s("oa_qwen_audio_weights_load_gguf", vp, C.c_char_p, C.c_char_p, C.c_size_t)
    s("oa_qwen_audio_weights_config", None, vp, C.POINTER(QwenAudioConfig))
    s("oa_qwen_audio_encoder_create", vp, vp, vp)
    s("oa_qwen_audio_encoder_free", None, vp)
    s("oa_qwen_audio_encode", i, vp, vp, i, vp, C.POINTER(C.c_double))
    s("oa_qwen_audio_encoder_set_flash_attention_precision", i, vp, i)
    s("oa_classify_quant_tensor_role", i, vp, i, i, i, i)
    s("oa_quant_target_write_type", i, vp, i, i, i, i)
    s("oa_qwen_decode_graph", vp, vp)
    _lib = L
    return L


class QwenWeights:
    """Host bytes of a Qwen3-shaped decoder: synthesised (seeded N(0, 0.02),
    quantized), or views into a mapped qwen3-asr runtime pack (load_gguf)."""

    def __init__(self, wtype: int, seed: int = 1234, rope_theta: float = 1e6, rms_eps: float = 1e-6, **shape):
        self.cfg = QwenConfig(rope_theta=rope_theta, rms_eps=rms_eps, wtype=wtype, seed=seed, **shape)
        # every matrix must be stored as the pack writer's policy stores it
        # for this rung (a Q4_K pack keeps Q8_0 where ne0 % 256 != 0)
        c = self.cfg
        q_w = c.n_head * c.head_dim
        for name, dims, role in (("token_embd", (c.d_model, c.vocab), ROLE_EMBEDDING_TABLE),
                                 ("attn_q/k/v", (c.d_model, q_w), ROLE_TEXT_DECODER_MATRIX),
                                 ("attn_output", (q_w, c.d_model), ROLE_TEXT_DECODER_MATRIX),
                                 ("ffn_gate/up", (c.d_model, c.ffn), ROLE_TEXT_DECODER_MATRIX),
                                 ("ffn_down", (c.ffn, c.d_model), ROLE_TEXT_DECODER_MATRIX)):
            got = target_write_type(dims, pack_rung(wtype), role)
            if got != wtype:
                raise ValueError(f"{name} {dims}: a {PACK_LABELS[pack_rung(wtype)]} pack stores it as ggml type "
                                 f"{got}, not {wtype}")
        self.ptr = lib().oa_qwen_weights_synthesize(C.byref(self.cfg))
        if not self.ptr:
            raise RuntimeError("weight synthesis failed")

    @classmethod
    def load_gguf(cls, path) -> "QwenWeights":
        err = C.create_string_buffer(512)
        ptr = lib().oa_qwen_weights_load_gguf(str(path).encode(), err, len(err))
        if not ptr:
            raise ValueError(f"{path}: {err.value.decode()}")
        self = cls.__new__(cls)
        self.ptr = ptr
        self.cfg = QwenConfig()
        lib().oa_qwen_weights_config(ptr, C.byref(self.cfg))
        return self

    def array(self, layer: int, kind: int) -> np.ndarray:
        """a copy of one tensor's host bytes (uint8)"""
        p, n = self.tensor(layer, kind)
        if not p:
            return None
        return np.ctypeslib.as_array((C.c_uint8 * n).from_address(p)).copy()

    def tensor(self, layer: int, kind: int) -> tuple[int, int]:
        n = C.c_size_t(0)
        p = lib().oa_qwen_weights_tensor(self.ptr, layer, kind, C.byref(n))
        return p, n.value

    def pointer_table(self) -> list[int]:
        """[tok_embd, out_norm, per layer: attn_norm, qkv, q_norm, k_norm, o, ffn_norm, gate, up, down,
        then the separate output projection or None when tied]"""
        t = [self.tensor(-1, TOKEN_EMBD)[0], self.tensor(-1, OUTPUT_NORM)[0]]
        for layer in range(self.cfg.n_layers):
            t += [self.tensor(layer, k)[0] for k in LAYER_KINDS]
        return t + [self.tensor(-1, OUTPUT)[0]]

    def free(self):
        if self.ptr:
            lib().oa_qwen_weights_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class QwenModel:
    def __init__(self, weights: QwenWeights, backend):
        self.weights = weights
        self.cfg = weights.cfg
        self.ptr = lib().oa_qwen_model_create(backend, weights.ptr)
        if not self.ptr:
            raise RuntimeError("model upload failed")

    def session(self, n_seq: int, max_positions: int) -> "QwenSession":
        return QwenSession(self, n_seq, max_positions)

    def free(self):
        if self.ptr:
            lib().oa_qwen_model_free(self.ptr)
            self.ptr = None


class QwenSession:
    def __init__(self, model: QwenModel, n_seq: int, max_positions: int):
        self.model = model
        self.n_seq = n_seq
        self.max_positions = max_positions
        self.ptr = lib().oa_qwen_session_create(model.ptr, n_seq, max_positions)
        if not self.ptr:
            raise RuntimeError("session (KV arena) allocation failed")

    def _check(self, st: int, what: str):
        if st != 0:
            raise RuntimeError(f"{what} failed with ggml status {st}")

    def prefill_embeddings(self, emb: np.ndarray) -> np.ndarray:
        emb = np.ascontiguousarray(emb, dtype=np.float32)  # [n_seq, T, d]
        top1 = np.zeros(self.n_seq, np.int32)
        self._check(lib().oa_qwen_prefill_embeddings(self.ptr, emb.ctypes.data, emb.shape[1], top1.ctypes.data),
                    "prefill (embeddings)")
        return top1

    def prefill_tokens(self, tokens: np.ndarray) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)  # [n_seq, T]
        top1 = np.zeros(self.n_seq, np.int32)
        self._check(lib().oa_qwen_prefill_tokens(self.ptr, tokens.ctypes.data, tokens.shape[1], top1.ctypes.data),
                    "prefill (tokens)")
        return top1

    def step(self, tokens: np.ndarray, want_logits: bool = False):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        top1 = np.zeros(self.n_seq, np.int32)
        logits = np.zeros((self.n_seq, self.model.cfg.vocab), np.float32) if want_logits else None
        self._check(lib().oa_qwen_decode_step(self.ptr, tokens.ctypes.data, top1.ctypes.data,
                                              logits.ctypes.data if want_logits else None), "decode step")
        return (top1, logits) if want_logits else top1

    def generate(self, first: np.ndarray, n_steps: int):
        first = np.ascontiguousarray(first, dtype=np.int32)
        out = np.zeros((n_steps, self.n_seq), np.int32)
        ms = np.zeros(n_steps, np.float64)
        self._check(lib().oa_qwen_generate(self.ptr, first.ctypes.data, n_steps, out.ctypes.data, ms.ctypes.data),
                    "generate")
        return out, ms

    def read_kv(self, layer: int, seq: int):
        c = self.model.cfg
        shape = (c.n_kv_head, self.max_positions, c.head_dim)
        k = np.zeros(shape, np.uint16)
        v = np.zeros(shape, np.uint16)
        self._check(lib().oa_qwen_read_kv(self.ptr, layer, seq, k.ctypes.data, v.ctypes.data), "read_kv")
        return k, v

    def decode_graph(self):
        return lib().oa_qwen_decode_graph(self.ptr)

    def position(self, seq: int = 0) -> int:
        return lib().oa_qwen_session_position(self.ptr, seq)

    def set_flash_attention_precision(self, precision: int):
        """the self-attention's contract (set_flash_attention_precision,
        llm_transformer.rs:3044-3053): GGML_PREC_DEFAULT runs prefill chunks
        on the matrix cores and, where it is planned, the decode step in the
        single-query workgroup form, within float tolerance; GGML_PREC_F32
        keeps the exact chunked form"""
        self._check(lib().oa_qwen_session_set_flash_attention_precision(self.ptr, int(precision)),
                    "set_flash_attention_precision")

    def set_matmul_precision(self, precision: int):
        """the quantized projections' MUL_MAT precision (the graph's
        GgmlMatmulPrecision, cpu_graph.rs:142-146, 3624-3685): GGML_PREC_DEFAULT
        runs wide prefill products on the f16 matrix cores within float
        tolerance, GGML_PREC_F32 keeps every product exact"""
        self._check(lib().oa_qwen_session_set_matmul_precision(self.ptr, int(precision)), "set_matmul_precision")

    def set_reversed_top1(self, enable: bool = True):
        """greedy top-1 through the reversed-row GET_ROWS + ARGMAX graph"""
        lib().oa_qwen_session_set_reversed_top1(self.ptr, int(enable))

    def set_hip_lane(self, enable: bool = True, prefill_chunk: int = 256):
        """step graphs as the unmodified host builds them on a discrete-GPU
        HIP backend: REPEAT-expanded K/V (expand_attention_kv), the unfused
        attention chain for prefill chunks of more than two positions, even
        prefill chunks of at most prefill_chunk positions (one sequence)"""
        self._check(lib().oa_qwen_session_set_hip_lane(self.ptr, int(enable), int(prefill_chunk)), "set_hip_lane")

    def free(self):
        if self.ptr:
            lib().oa_qwen_session_free(self.ptr)
            self.ptr = None


class WhisperWeights:
    """Whisper decoder weights (host bytes, Q8_0 matrices): synthesised, or
    views into a mapped whisper runtime pack (load_gguf)."""

    def __init__(self, seed: int = 1234, ln_eps: float = 1e-5, ffn_act: int = FFN_GELU, **shape):
        self.cfg = WhisperConfig(shape["d_model"], shape["n_layers"], shape["n_head"], shape["ffn"], shape["vocab"],
                                 shape["max_positions"], shape["n_frames"], ln_eps, seed, ffn_act)
        self.ptr = lib().oa_whisper_weights_synthesize(C.byref(self.cfg))
        if not self.ptr:
            raise RuntimeError("whisper weight synthesis failed")

    @classmethod
    def load_gguf(cls, path) -> "WhisperWeights":
        err = C.create_string_buffer(512)
        ptr = lib().oa_whisper_weights_load_gguf(str(path).encode(), err, len(err))
        if not ptr:
            raise ValueError(f"{path}: {err.value.decode()}")
        self = cls.__new__(cls)
        self.ptr = ptr
        self.cfg = WhisperConfig()
        lib().oa_whisper_weights_config(ptr, C.byref(self.cfg))
        return self

    def tensor_ptr(self, layer: int, kind: int) -> int:
        n = C.c_size_t(0)
        p = lib().oa_whisper_weights_tensor(self.ptr, layer, kind, C.byref(n))
        if not p:
            raise KeyError((layer, kind))
        return p

    def array(self, layer: int, kind: int) -> np.ndarray:
        """a copy of one tensor's host bytes (uint8)"""
        n = C.c_size_t(0)
        p = lib().oa_whisper_weights_tensor(self.ptr, layer, kind, C.byref(n))
        if not p:
            raise KeyError((layer, kind))
        return np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p)).copy()

    def pointer_table(self):
        """per layer the 24 tensors in kind order, then token embedding,
        position embedding, final LayerNorm weight and bias (oracle order)"""
        out = [self.tensor_ptr(l, k) for l in range(self.cfg.n_layers) for k in range(WH_LAYER_KINDS)]
        out += [self.tensor_ptr(-1, k) for k in (WH_TOKEN_EMBD, WH_POS_EMBD, WH_FINAL_LN_W, WH_FINAL_LN_B)]
        return out

    def free(self):
        if self.ptr:
            lib().oa_whisper_weights_free(self.ptr)
            self.ptr = None


class WhisperModel:
    def __init__(self, weights: WhisperWeights, backend):
        self.cfg = weights.cfg
        self.ptr = lib().oa_whisper_model_create(backend, weights.ptr)
        if not self.ptr:
            raise RuntimeError("whisper model upload failed")

    def session(self) -> "WhisperSession":
        return WhisperSession(self)

    def free(self):
        if self.ptr:
            lib().oa_whisper_model_free(self.ptr)
            self.ptr = None


class WhisperSession:
    """Batch-1 Whisper decode: cross K/V from encoder states, then greedy steps."""

    def __init__(self, model: WhisperModel):
        self.model = model
        self.ptr = lib().oa_whisper_session_create(model.ptr)
        if not self.ptr:
            raise RuntimeError("whisper session allocation failed")

    @staticmethod
    def _check(st: int, what: str):
        if st != 0:
            raise RuntimeError(f"{what} failed with ggml status {st}")

    def set_encoder(self, enc: np.ndarray):
        enc = np.ascontiguousarray(enc, dtype=np.float32)
        self._check(lib().oa_whisper_set_encoder(self.ptr, enc.ctypes.data), "cross K/V precompute")

    def step(self, token: int, want_logits: bool = False):
        top1 = C.c_int32(0)
        logits = np.zeros(self.model.cfg.vocab, np.float32) if want_logits else None
        self._check(lib().oa_whisper_decode_step(self.ptr, int(token), C.byref(top1),
                                                 logits.ctypes.data if want_logits else None), "whisper step")
        return (top1.value, logits) if want_logits else top1.value

    def generate(self, first: int, n_steps: int):
        out = np.zeros(n_steps, np.int32)
        ms = np.zeros(n_steps, np.float64)
        self._check(lib().oa_whisper_generate(self.ptr, int(first), n_steps, out.ctypes.data, ms.ctypes.data),
                    "whisper generate")
        return out, ms

    def read_cross(self, layer: int):
        c = self.model.cfg
        k = np.zeros((c.n_frames, c.d_model), np.uint16)
        v = np.zeros((c.n_frames, c.d_model), np.uint16)
        self._check(lib().oa_whisper_read_cross(self.ptr, layer, k.ctypes.data, v.ctypes.data), "read_cross")
        return k, v

    def read_self(self, layer: int):
        """the layer's self-attention K / V caches, f16 bits [max_positions, d_model]"""
        c = self.model.cfg
        k = np.zeros((c.max_positions, c.d_model), np.uint16)
        v = np.zeros((c.max_positions, c.d_model), np.uint16)
        self._check(lib().oa_whisper_read_self(self.ptr, layer, k.ctypes.data, v.ctypes.data), "read_self")
        return k, v

    def decode_graph(self):
        return lib().oa_whisper_decode_graph(self.ptr)

    def set_flash_attention_precision(self, precision: int):
        """the self and cross attention's contract (the seq2seq decoder
        graphs' flash_attention_precision, nn/decoder.rs:3064-3728):
        GGML_PREC_DEFAULT (the default) or GGML_PREC_F32 (the exact chunked
        form)"""
        self._check(lib().oa_whisper_session_set_flash_attention_precision(self.ptr, int(precision)),
                    "set_flash_attention_precision")

    def position(self) -> int:
        return lib().oa_whisper_session_position(self.ptr)

    def free(self):
        if self.ptr:
            lib().oa_whisper_session_free(self.ptr)
            self.ptr = None


def whisper_inputs(shape: dict, n_prompt: int = 4, seed: int = 91):
    """seeded N(0,1) encoder states [n_frames, d] and prompt token ids"""
    enc = g.synth_normal(seed, 3000, shape["n_frames"] * shape["d_model"]).reshape(shape["n_frames"], shape["d_model"])
    prompt = np.zeros(n_prompt, np.int32)
    g.base().oa_synth_uniform_i32(seed, 3001, n_prompt, shape["vocab"], prompt.ctypes.data)
    return enc, prompt


def detect_degenerate_ngram(tokens, max_ngram: int = 8, bound=None):
    """(keep_len, ngram_len, repeats) when the tail ends in a loop, else None.
    bound: a function of the cycle length (the reference's
    max_consecutive_repeats), or None for the shipped 8/6/4 tiers."""
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    n, r = C.c_int(0), C.c_int(0)
    table = None
    if bound is not None and max_ngram > 0:
        table = np.array([bound(k) for k in range(1, max_ngram + 1)], np.int32)
    keep = lib().oa_detect_degenerate_ngram(t.ctypes.data if t.size else None, len(t), max_ngram,
                                            table.ctypes.data if table is not None else None, C.byref(n), C.byref(r))
    return None if keep < 0 else (keep, n.value, r.value)


class QwenAudioWeights:
    """Host bytes of a Qwen3-ASR-shaped audio encoder, synthesised (seeded
    N(0, 0.02) projections of ggml type wtype, f32 conv kernels and vectors)."""

    def __init__(self, wtype: int = g.F16, seed: int = 4242, **shape):
        self.cfg = QwenAudioConfig(wtype=wtype, seed=seed, **shape)
        self.ptr = lib().oa_qwen_audio_weights_synthesize(C.byref(self.cfg))
        if not self.ptr:
            raise ValueError(f"audio encoder weights: shape {shape} does not fit type {wtype}")

    @classmethod
    def load_gguf(cls, path) -> "QwenAudioWeights":
        """the audio encoder of a qwen3-asr runtime pack (oa_qwen_audio_weights_load_gguf)"""
        err = C.create_string_buffer(512)
        ptr = lib().oa_qwen_audio_weights_load_gguf(str(path).encode(), err, len(err))
        if not ptr:
            raise ValueError(f"{path}: {err.value.decode()}")
        self = cls.__new__(cls)
        self.ptr = ptr
        self.cfg = QwenAudioConfig()
        lib().oa_qwen_audio_weights_config(ptr, C.byref(self.cfg))
        return self

    def array(self, layer: int, kind: int) -> np.ndarray:
        """a copy of one tensor's bytes (uint8); layer -1 for the global tensors"""
        n = C.c_size_t(0)
        p = lib().oa_qwen_audio_weights_tensor(self.ptr, layer, kind, C.byref(n))
        if not p:
            return None
        return np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p)).copy()

    def free(self):
        if self.ptr:
            lib().oa_qwen_audio_weights_free(self.ptr)
            self.ptr = None


def qwen_audio_token_count(n_frames: int) -> int:
    return int(lib().oa_qwen_audio_token_count(n_frames))


class QwenAudioEncoder:
    """The audio encoder graph on a backend (oa_qwen_audio_encoder_create)."""

    def __init__(self, weights: QwenAudioWeights, backend):
        self.cfg = weights.cfg
        self.ptr = lib().oa_qwen_audio_encoder_create(backend, weights.ptr)
        if not self.ptr:
            raise RuntimeError("audio encoder: weight upload failed")

    def encode(self, mel: np.ndarray):
        """mel [n_mels, n_frames] -> (embeddings [rows, out_dim], compute ms)"""
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        n_frames = mel.shape[1]
        out = np.zeros((qwen_audio_token_count(n_frames), self.cfg.out_dim), np.float32)
        ms = C.c_double(0.0)
        st = lib().oa_qwen_audio_encode(self.ptr, mel.ctypes.data, n_frames, out.ctypes.data, C.byref(ms))
        if st != 0:
            raise RuntimeError(f"audio encode failed: status {st}")
        return out, ms.value

    def set_flash_attention_precision(self, precision: int):
        """GGML_PREC_DEFAULT (as the reference builds the encoder) or
        GGML_PREC_F32 (the exact chunked attention)"""
        if lib().oa_qwen_audio_encoder_set_flash_attention_precision(self.ptr, int(precision)) != 0:
            raise ValueError(f"unknown flash-attention precision {precision}")

    def free(self):
        if self.ptr:
            lib().oa_qwen_audio_encoder_free(self.ptr)
            self.ptr = None


# pack storage policy (crates/openasr-core/src/models/pack_quant.rs):
# requested rungs, tensor roles, quantized axes
PACK_FP16, PACK_Q8_0, PACK_Q3_K, PACK_Q4_K = range(4)
(ROLE_ACOUSTIC_ENCODER_MATRIX, ROLE_TEXT_DECODER_MATRIX, ROLE_EMBEDDING_TABLE, ROLE_OUTPUT_PROJECTION,
 ROLE_PRECISION_CRITICAL_MATRIX, ROLE_NON_QUANTIZABLE) = range(6)
AXIS_FIRST, AXIS_LAST = range(2)
PACK_LABELS = {PACK_FP16: "fp16", PACK_Q8_0: "q8_0", PACK_Q3_K: "q3_k", PACK_Q4_K: "q4_k"}
GGML_Q3_K = 11


def _policy(fn, dims, quantization: int, role: int, axis: int):
    d = np.ascontiguousarray(dims, dtype=np.uint64)
    r = fn(d.ctypes.data if d.size else None, int(d.size), quantization, role, axis)
    if r == -2:
        raise ValueError(f"pack policy: argument out of range (quantization {quantization}, role {role}, axis {axis})")
    return None if r < 0 else r


def classify_quant_tensor_role(dims, quantization: int, role: int, axis: int = AXIS_FIRST):
    """classify_quant_tensor_role (pack_quant.rs:179-213): the ggml type a
    tensor of this role and shape is written as for the requested rung, or
    None (kept in the rung's non-quantized representation)."""
    return _policy(lib().oa_classify_quant_tensor_role, dims, quantization, role, axis)


def target_write_type(dims, quantization: int, role: int, axis: int = AXIS_FIRST):
    """target_write_type (pack_quant.rs:127-147) for a resolved role: only
    rank-2 tensors are block-quantized. role None (a contract with no
    acoustic encoder) writes nothing quantized."""
    if role is None:
        return None
    return _policy(lib().oa_quant_target_write_type, dims, quantization, role, axis)


def pack_rung(wtype: int) -> int:
    """the pack rung that asks for weights of ggml type wtype"""
    return {g.Q8_0: PACK_Q8_0, g.Q4_K: PACK_Q4_K}[wtype]


@dataclass
class QwenWorkload:
    """One of the decode configurations the path is measured on."""
    name: str
    shape: dict
    wtype: int
    n_seq: int
    prefix: int          # audio-embedding prefix positions, N(0,1)
    prompt: int          # prompt tokens after the prefix
    decode: int          # greedy tokens
    max_positions: int


WORKLOADS = {
    "qwen3-0.6b-q8_0-b1": QwenWorkload("qwen3-0.6b-q8_0-b1", QWEN3_06B, g.Q8_0, 1, 375, 8, 256, 1024),
    "qwen3-0.6b-q4_K-b8": QwenWorkload("qwen3-0.6b-q4_K-b8", QWEN3_06B, g.Q4_K, 8, 375, 8, 512, 1024),
    "qwen3-1.7b-q4_K-b8": QwenWorkload("qwen3-1.7b-q4_K-b8", QWEN3_17B, g.Q4_K, 8, 3000, 8, 1024, 4096),
}


def workload_inputs(w: QwenWorkload, seed: int = 77):
    """seeded N(0,1) prefixes [n_seq, prefix, d] and prompt ids [n_seq, prompt]"""
    d = w.shape["d_model"]
    emb = np.stack([g.synth_normal(seed, 1000 + s, w.prefix * d).reshape(w.prefix, d) for s in range(w.n_seq)])
    prompt = np.zeros((w.n_seq, w.prompt), np.int32)
    for s in range(w.n_seq):
        g.base().oa_synth_uniform_i32(seed, 2000 + s, w.prompt, w.shape["vocab"], prompt[s].ctypes.data)
    return emb, prompt
