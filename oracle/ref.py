"""numpy wrapper of the CPU oracle (oracle/ggml_cpu_ref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product never imports it.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "build" / "libggml_cpu_ref.so"

F32, F16, Q8_0, Q3_K, Q4_K, Q8_K = 0, 1, 8, 11, 12, 15
BLOCK = {Q8_0: (32, 34), Q3_K: (256, 110), Q4_K: (256, 144), Q8_K: (256, 292)}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} missing: run `python -m openasr_amd.build`")
    L = C.CDLL(str(LIB_PATH))
    vp, i64, f, i = C.c_void_p, C.c_int64, C.c_float, C.c_int

    def s(name, res, *args):
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = list(args)

    s("ref_fp32_to_fp16", C.c_uint16, f)
    s("ref_fp16_to_fp32", f, C.c_uint16)
    for n in ("ref_quantize_row_q8_0_weights", "ref_quantize_row_q4_K", "ref_quantize_row_q8_0_act",
              "ref_quantize_row_q8_K", "ref_dequantize_row_q8_0", "ref_dequantize_row_q4_K",
              "ref_dequantize_row_q8_K", "ref_dequantize_row_q3_K"):
        s(n, None, vp, vp, i64)
    s("ref_vec_dot_q8_0_q8_0", f, i64, vp, vp)
    s("ref_vec_dot_q4_K_q8_K", f, i64, vp, vp)
    s("ref_vec_dot_q3_K_q8_K", f, i64, vp, vp)
    s("ref_q3_K_scale", i, vp, i)
    s("ref_vec_dot_f16", f, i64, vp, vp)
    s("ref_row_size", C.c_size_t, i, i64)
    s("ref_mul_mat", None, i, vp, C.c_size_t, i64, i64, vp, i64, i64, vp, i64, i)
    s("ref_rms_norm", None, vp, vp, i64, i64, f)
    s("ref_norm", None, vp, vp, i64, i64, f)
    s("ref_silu", f, f)
    s("ref_gelu", f, f)
    s("ref_gelu_f32", f, f)
    s("ref_rope_neox", None, vp, vp, i64, i64, i64, vp, i, f, f)
    s("ref_soft_max_ext", None, vp, vp, vp, i64, i64, f)
    s("ref_argmax_last", C.c_int32, vp, i64)
    s("ref_argmax_first", C.c_int32, vp, i64)
    s("ref_expf_det", f, f)
    s("ref_erff_det", f, f)
    s("ref_erf_coef", C.c_double, C.c_int)
    s("ref_gelu_erf", f, f)
    s("ref_relu", f, f)
    s("ref_sincosf_det", None, f, vp, vp)
    s("ref_flash_attn_ext", None, vp, i64, i64, vp, vp, i64, i64, vp, i64, vp, i64, i64, i64, i64, i64, f, i, i)
    s("ref_naive_attention", None, vp, i64, i64, vp, vp, i64, i64, vp, i64, vp, i64, i64, i64, i64, i64, f, i, i)
    _lib = L
    return L


def _p(a: np.ndarray):
    return a.ctypes.data


def row_size(typ: int, k: int) -> int:
    return int(lib().ref_row_size(typ, k))


def quantize_weights(typ: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    out = np.zeros(rows * row_size(typ, k), dtype=np.uint8)
    fn = lib().ref_quantize_row_q8_0_weights if typ == Q8_0 else lib().ref_quantize_row_q4_K
    fn(_p(x), _p(out), rows * k)
    return out


def quantize_act(typ: int, x: np.ndarray) -> np.ndarray:
    """activation side: Q8_0 (x86 ggml-cpu rule) or Q8_K"""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(row_size(typ, x.size), dtype=np.uint8)
    fn = lib().ref_quantize_row_q8_0_act if typ == Q8_0 else lib().ref_quantize_row_q8_K
    fn(_p(x), _p(out), x.size)
    return out


def dequantize(typ: int, q: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    fn = {Q8_0: lib().ref_dequantize_row_q8_0, Q4_K: lib().ref_dequantize_row_q4_K,
          Q8_K: lib().ref_dequantize_row_q8_K, Q3_K: lib().ref_dequantize_row_q3_K}[typ]
    q = np.ascontiguousarray(q)
    fn(_p(q), _p(out), n)
    return out


def mul_mat(wtype: int, w: np.ndarray, m: int, k: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """x: [n, k] f32 -> [n, m] f32 (ggml dst layout ne=[m, n])"""
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[0]
    dst = np.zeros((n, m), dtype=np.float32)
    rb = row_size(wtype, k) if wtype in (Q8_0, Q3_K, Q4_K) else (2 * k if wtype == F16 else 4 * k)
    lib().ref_mul_mat(wtype, _p(w), rb, m, k, _p(x), k, n, _p(dst), m, threads)
    return dst


def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().ref_rms_norm(_p(x), _p(y), x.shape[-1], x.size // x.shape[-1], eps)
    return y


def norm(x: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().ref_norm(_p(x), _p(y), x.shape[-1], x.size // x.shape[-1], eps)
    return y


def silu(x: np.ndarray) -> np.ndarray:
    f = lib().ref_silu
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).reshape(-1)], np.float32).reshape(np.shape(x))


def gelu(x: np.ndarray) -> np.ndarray:
    f = lib().ref_gelu
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).reshape(-1)], np.float32).reshape(np.shape(x))


def rope_neox(x: np.ndarray, pos: np.ndarray, n_dims: int, freq_base: float, freq_scale: float = 1.0):
    """x: [tokens, heads, head_dim]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    t, h, d = x.shape
    y = np.empty_like(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    lib().ref_rope_neox(_p(x), _p(y), d, h, t, _p(pos), n_dims, freq_base, freq_scale)
    return y


def soft_max_ext(x: np.ndarray, mask_f16: np.ndarray | None, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    m = None if mask_f16 is None else np.ascontiguousarray(mask_f16, dtype=np.uint16)
    lib().ref_soft_max_ext(_p(x), None if m is None else _p(m), _p(y), x.shape[-1], x.size // x.shape[-1], scale)
    return y


def argmax_last(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().ref_argmax_last(_p(x), x.size))


def argmax_first(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().ref_argmax_first(_p(x), x.size))


def flash_attn(q: np.ndarray, k16: np.ndarray, v16: np.ndarray, mask16: np.ndarray | None, scale: float,
               fidelity: int = 1, threads: int = 0) -> np.ndarray:
    """q: [n_q, Hq, D] f32; k16, v16: [Hkv, n_kv, D] f16 bits; mask16: [n_q, n_kv] f16 bits.
    fidelity 1: ggml-cpu numerics (f16 Q, f16 V accumulator); 2: f16 Q, f32
    online accumulation; 0: f32 throughout; 3: f16 Q, two-pass f64 sums over
    the whole span; 4: f16 Q, fixed 64-position chunks with their own maxima
    and f64 sums, combined in chunk order; 5: the chunks of 4 with f32 fma
    chains in a fixed order inside each chunk (scores over dims, p*V over
    positions) and the f64 chunk combine (the device's definition). Returns
    [n_q, Hq, D] f32."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k16 = np.ascontiguousarray(k16, dtype=np.uint16)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    n_q, hq, d = q.shape
    hkv, n_kv, _ = k16.shape
    out = np.zeros((n_q, hq, d), dtype=np.float32)
    m = None if mask16 is None else np.ascontiguousarray(mask16, dtype=np.uint16)
    lib().ref_flash_attn_ext(_p(q), hq * d, d, _p(k16), _p(v16), n_kv * d, d, None if m is None else _p(m),
                             0 if m is None else m.shape[-1], _p(out), d, n_q, hq, hkv, n_kv, scale,
                             int(fidelity), threads)
    return out


def naive_attention(q: np.ndarray, k16: np.ndarray, v16: np.ndarray, mask16: np.ndarray | None, scale: float,
                    prec_f32: bool = True, threads: int = 0) -> np.ndarray:
    """The unfused attention chain (MUL_MAT(K, Q) -> SOFT_MAX_EXT -> MUL_MAT of
    V^T by P -> PERMUTE/CONT, nn/decoder.rs:2154-2200) in the oracle's fixed
    order; layouts as flash_attn. prec_f32: GGML_PREC_F32 on both products
    (Q and P kept f32), else both rounded to f16. Returns [n_q, Hq, D] f32."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k16 = np.ascontiguousarray(k16, dtype=np.uint16)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    n_q, hq, d = q.shape
    hkv, n_kv, _ = k16.shape
    out = np.zeros((n_q, hq, d), dtype=np.float32)
    m = None if mask16 is None else np.ascontiguousarray(mask16, dtype=np.uint16)
    lib().ref_naive_attention(_p(q), hq * d, d, _p(k16), _p(v16), n_kv * d, d, None if m is None else _p(m),
                              0 if m is None else m.shape[-1], _p(out), d, n_q, hq, hkv, n_kv, scale,
                              int(bool(prec_f32)), threads)
    return out


# ------------------------------------------------------------ decoders ---

class QwenDims(C.Structure):
    _fields_ = [("d_model", C.c_int), ("n_layers", C.c_int), ("n_head", C.c_int), ("n_kv_head", C.c_int),
                ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("wtype", C.c_int),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float), ("out_wtype", C.c_int)]


class QwenRef:
    """CPU reference of one Qwen3 decoder sequence over host weight bytes
    (a pointer table into the same buffers the device was loaded from)."""

    def __init__(self, cfg, pointer_table, max_pos: int, fa_fidelity: int = 5, threads: int = 0):
        L = lib()
        L.ref_qwen_forward.restype = C.c_int32
        L.ref_qwen_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                       C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int]
        L.ref_qwen_embed.restype = None
        L.ref_qwen_embed.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
        self.dims = QwenDims(cfg.d_model, cfg.n_layers, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.ffn, cfg.vocab,
                             cfg.wtype, cfg.rope_theta, cfg.rms_eps, getattr(cfg, "out_wtype", 0))
        self.table = (C.c_void_p * len(pointer_table))(*pointer_table)
        self.max_pos = max_pos
        self.fidelity = fa_fidelity
        self.threads = threads
        shape = (cfg.n_kv_head, max_pos, cfg.head_dim)
        self.k = [np.zeros(shape, np.uint16) for _ in range(cfg.n_layers)]
        self.v = [np.zeros(shape, np.uint16) for _ in range(cfg.n_layers)]
        self.kp = (C.c_void_p * cfg.n_layers)(*[a.ctypes.data for a in self.k])
        self.vp = (C.c_void_p * cfg.n_layers)(*[a.ctypes.data for a in self.v])
        self.pos = 0

    def embed(self, tokens) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros((len(tokens), self.dims.d_model), np.float32)
        lib().ref_qwen_embed(C.byref(self.dims), self.table, tokens.ctypes.data, len(tokens), out.ctypes.data)
        return out

    def forward(self, x: np.ndarray):
        """x [T, d] layer-0 input at the next T positions -> (top1, logits of the last position)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        logits = np.zeros(self.dims.vocab, np.float32)
        top1 = lib().ref_qwen_forward(C.byref(self.dims), self.table, self.kp, self.vp, self.max_pos,
                                      x.ctypes.data, x.shape[0], self.pos, logits.ctypes.data, self.fidelity,
                                      self.threads)
        self.pos += x.shape[0]
        return int(top1), logits

    def step(self, token: int):
        return self.forward(self.embed([token]))

    def prefill_hip_lane(self, x: np.ndarray, chunk: int):
        """x [T, d] through the chunks of the unmodified host's HIP-lane
        prefill (even widths of at most `chunk`, an odd width above one
        trimmed by one, llm_transformer.rs:7903-7911): the unfused attention
        chain with GGML_PREC_F32 (fidelity 6) for chunks of more than two
        positions over a span of more than 32 (llm_transformer.rs:7864-7877),
        the flash attention definition otherwise. Returns the last chunk's
        (top1, logits)."""
        t0, res = 0, None
        keep = self.fidelity
        try:
            while t0 < len(x):
                w = min(chunk, len(x) - t0)
                if w > 1 and w % 2:
                    w -= 1
                self.fidelity = 6 if w > 2 and self.max_pos > 32 else keep
                res = self.forward(x[t0:t0 + w])
                t0 += w
        finally:
            self.fidelity = keep
        return res


class QwenRefBatch:
    """CPU reference of a batched decode step over n_seq sequences (weights
    streamed once per step), continuing from given KV caches."""

    def __init__(self, cfg, pointer_table, max_pos: int, n_seq: int, fa_fidelity: int = 5, threads: int = 0):
        L = lib()
        L.ref_qwen_decode_batch.restype = None
        L.ref_qwen_decode_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                            C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        self.dims = QwenDims(cfg.d_model, cfg.n_layers, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.ffn, cfg.vocab,
                             cfg.wtype, cfg.rope_theta, cfg.rms_eps, getattr(cfg, "out_wtype", 0))
        self.table = (C.c_void_p * len(pointer_table))(*pointer_table)
        self.max_pos, self.n_seq, self.fidelity, self.threads = max_pos, n_seq, fa_fidelity, threads
        shape = (cfg.n_kv_head, max_pos, cfg.head_dim)
        self.k = [[np.zeros(shape, np.uint16) for _ in range(cfg.n_layers)] for _ in range(n_seq)]
        self.v = [[np.zeros(shape, np.uint16) for _ in range(cfg.n_layers)] for _ in range(n_seq)]
        flat_k = [a.ctypes.data for s in self.k for a in s]
        flat_v = [a.ctypes.data for s in self.v for a in s]
        self.kp = (C.c_void_p * len(flat_k))(*flat_k)
        self.vp = (C.c_void_p * len(flat_v))(*flat_v)
        self.pos = np.zeros(n_seq, np.int32)

    def step(self, tokens, want_logits: bool = False):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        top1 = np.zeros(self.n_seq, np.int32)
        logits = np.zeros((self.n_seq, self.dims.vocab), np.float32) if want_logits else None
        pos = np.ascontiguousarray(self.pos, dtype=np.int32)
        lib().ref_qwen_decode_batch(C.byref(self.dims), self.table, self.kp, self.vp, self.max_pos,
                                    tokens.ctypes.data, pos.ctypes.data, self.n_seq, top1.ctypes.data,
                                    logits.ctypes.data if want_logits else None, self.fidelity, self.threads)
        self.pos += 1
        return (top1, logits) if want_logits else top1


class QwenFastBatch(QwenRefBatch):
    """The benchmark's CPU baseline leg (oracle/cpu_fast.c): the same batched
    decode step with ggml-cpu's arithmetic classes on the host ISA (VNNI or
    AVX2 int8 block dots with f32 accumulation, f16 V accumulator in
    attention). Not the checker: tests/test_cpu_fast.py holds it to the
    oracle within float tolerance."""

    def __init__(self, cfg, pointer_table, max_pos: int, n_seq: int, threads: int = 0):
        super().__init__(cfg, pointer_table, max_pos, n_seq, threads=threads)
        L = lib()
        L.fast_qwen_decode_batch.restype = None
        L.fast_qwen_decode_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                             C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int]

    def step(self, tokens, want_logits: bool = False):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        top1 = np.zeros(self.n_seq, np.int32)
        logits = np.zeros((self.n_seq, self.dims.vocab), np.float32) if want_logits else None
        pos = np.ascontiguousarray(self.pos, dtype=np.int32)
        lib().fast_qwen_decode_batch(C.byref(self.dims), self.table, self.kp, self.vp, self.max_pos,
                                     tokens.ctypes.data, pos.ctypes.data, self.n_seq, top1.ctypes.data,
                                     logits.ctypes.data if want_logits else None, self.threads)
        self.pos += 1
        return (top1, logits) if want_logits else top1


def fast_uses_vnni() -> bool:
    L = lib()
    L.fast_cpu_uses_vnni.restype = C.c_int
    return bool(L.fast_cpu_uses_vnni())


def fast_mul_mat(wtype: int, w_bytes: np.ndarray, m: int, k: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """the baseline leg's MUL_MAT: [n, m] f32 from weights of wtype and x [n, k]"""
    L = lib()
    L.fast_mul_mat.restype = None
    i64 = C.c_int64
    L.fast_mul_mat.argtypes = [C.c_int, C.c_void_p, C.c_size_t, i64, i64, C.c_void_p, i64, i64, C.c_void_p, i64,
                               C.c_int]
    x = np.ascontiguousarray(x, dtype=np.float32)
    w_bytes = np.ascontiguousarray(w_bytes)
    n = x.shape[0]
    out = np.zeros((n, m), np.float32)
    L.fast_mul_mat(wtype, w_bytes.ctypes.data, row_size(wtype, k), m, k, x.ctypes.data, k, n, out.ctypes.data, m,
                   threads)
    return out


def fast_attn_one(q: np.ndarray, k16: np.ndarray, v16: np.ndarray, mask16, scale: float) -> np.ndarray:
    """the baseline leg's decode attention for one query row: q [D] f32, k16 /
    v16 [n_kv, D] f16 bits, mask16 [n_kv] f16 bits or None"""
    L = lib()
    L.fast_attn_one.restype = None
    L.fast_attn_one.argtypes = [C.c_void_p] * 4 + [C.c_int64, C.c_int64, C.c_float, C.c_void_p]
    q = np.ascontiguousarray(q, dtype=np.float32)
    k16 = np.ascontiguousarray(k16, dtype=np.uint16)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    m = None if mask16 is None else np.ascontiguousarray(mask16, dtype=np.uint16)
    out = np.zeros(q.shape[-1], np.float32)
    L.fast_attn_one(_p(q), _p(k16), _p(v16), None if m is None else _p(m), k16.shape[0], q.shape[-1], scale, _p(out))
    return out


class WhisperDims(C.Structure):
    _fields_ = [("d_model", C.c_int), ("n_layers", C.c_int), ("n_head", C.c_int), ("ffn", C.c_int),
                ("vocab", C.c_int), ("max_positions", C.c_int), ("n_frames", C.c_int), ("ln_eps", C.c_float),
                ("ffn_act", C.c_int)]


class WhisperRef:
    """CPU reference of the Whisper decoder (batch 1) over host weight bytes:
    cross K/V precompute from encoder states, then one token per step."""

    def __init__(self, cfg, pointer_table, fa_fidelity: int = 5, threads: int = 0):
        L = lib()
        L.ref_whisper_cross_kv.restype = None
        L.ref_whisper_cross_kv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.ref_whisper_step.restype = C.c_int32
        L.ref_whisper_step.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_int32, C.c_int, C.c_void_p, C.c_int, C.c_int]
        self.dims = WhisperDims(cfg.d_model, cfg.n_layers, cfg.n_head, cfg.ffn, cfg.vocab, cfg.max_positions,
                                cfg.n_frames, cfg.ln_eps, getattr(cfg, "ffn_act", 0))
        self.table = (C.c_void_p * len(pointer_table))(*pointer_table)
        self.fidelity, self.threads = fa_fidelity, threads
        n = cfg.n_layers
        self.k = [np.zeros((cfg.max_positions, cfg.d_model), np.uint16) for _ in range(n)]
        self.v = [np.zeros((cfg.max_positions, cfg.d_model), np.uint16) for _ in range(n)]
        self.ck = [np.zeros((cfg.n_frames, cfg.d_model), np.uint16) for _ in range(n)]
        self.cv = [np.zeros((cfg.n_frames, cfg.d_model), np.uint16) for _ in range(n)]
        arr = lambda xs: (C.c_void_p * n)(*[a.ctypes.data for a in xs])
        self.kp, self.vp, self.ckp, self.cvp = arr(self.k), arr(self.v), arr(self.ck), arr(self.cv)
        self.pos = 0

    def set_encoder(self, enc: np.ndarray):
        enc = np.ascontiguousarray(enc, dtype=np.float32)
        lib().ref_whisper_cross_kv(C.byref(self.dims), self.table, enc.ctypes.data, self.ckp, self.cvp, self.threads)

    def step(self, token: int):
        logits = np.zeros(self.dims.vocab, np.float32)
        top1 = lib().ref_whisper_step(C.byref(self.dims), self.table, self.kp, self.vp, self.ckp, self.cvp,
                                      int(token), self.pos, logits.ctypes.data, self.fidelity, self.threads)
        self.pos += 1
        return int(top1), logits


def im2col(x: np.ndarray, kw: int, kh: int, s0: int, s1: int, p0: int, p1: int, d0: int, d1: int,
           is_2d: bool = True) -> np.ndarray:
    """ggml's IM2COL (f32 columns; the f16 result is these rounded to nearest
    even), the first half of ggml_conv_2d used by nn/conv.rs:82-110 /
    cpu_graph.rs:5191-5246 (the ggml-cpu kernel lives in the absent
    openasr-ggml fork; this restates ggml's published definition).
    x: [N, IC, IH, IW] (2-D) or [N, IC, IW] (1-D). Returns [N, OH, OW, IC*KH*KW]
    (1-D: [N, OW, IC*KW]); tap (ic, a, b) of output (oh, ow) reads input
    (oh*s1 + a*d1 - p1, ow*s0 + b*d0 - p0), zero outside the input."""
    if not is_2d:
        x, kh, s1, p1, d1 = x[:, :, None, :], 1, 1, 0, 1
    n, ic, ih, iw = x.shape
    oh = (ih + 2 * p1 - d1 * (kh - 1) - 1) // s1 + 1
    ow = (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1
    out = np.zeros((n, oh, ow, ic, kh, kw), np.float32)
    for a in range(kh):
        rows = np.arange(oh) * s1 + a * d1 - p1
        for b in range(kw):
            cols = np.arange(ow) * s0 + b * d0 - p0
            inside = ((rows >= 0) & (rows < ih))[:, None] & ((cols >= 0) & (cols < iw))[None, :]
            g = x[:, :, np.clip(rows, 0, ih - 1)][:, :, :, np.clip(cols, 0, iw - 1)]
            out[..., a, b] = np.where(inside[None, None], g, np.float32(0)).transpose(0, 2, 3, 1)
    return out.reshape(n, oh, ow, ic * kh * kw) if is_2d else out.reshape(n, ow, ic * kw)
