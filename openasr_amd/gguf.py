"""GGUF (v3) writer for OpenASR runtime packs (`.oasr` v1 = standard GGUF
bytes, docs/format/OASR_PACKAGE_CONTRACT_V1.md), the producer side of the
pack reader in libopenasr-models.so (oa_gguf_open). Mirrors what the
reference's pack writer emits (crates/openasr-core/src/ggml_runtime/
gguf_write.rs): typed metadata, tensor infos, then every tensor's bytes at the
pack's alignment.

`export_qwen_pack` writes a qwen3-asr LLM pack from decoder weights: the
hparam keys of arch/hparams.rs:52-58 and the tensor names of
models/qwen/decoder_contract.rs:686-705, 764-769, with the fused q|k|v
projection split back into attn_q / attn_k / attn_v. `export_whisper_pack`
writes the decoder part of a whisper pack: the keys of
models/whisper/runtime_contract.rs:180-230 and the tensor names of
models/whisper/ggml_tensor_binding.rs:135-210.
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
(U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64) = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


class GGUFWriter:
    """Collects metadata and tensors, then writes the file in one pass."""

    def __init__(self, alignment: int = 32):
        if alignment <= 0 or alignment & (alignment - 1):
            raise ValueError("alignment must be a power of two")
        self.alignment = alignment
        self.kv: list[tuple[str, int, object]] = []
        self.tensors: list[tuple[str, int, tuple[int, ...], bytes]] = []
        if alignment != 32:
            self.add("general.alignment", U32, alignment)

    def add(self, key: str, vtype: int, value) -> None:
        self.kv.append((key, vtype, value))

    def add_tensor(self, name: str, ggml_type: int, ne: tuple[int, ...], data: bytes | np.ndarray) -> None:
        """ne in ggml order (ne[0] = row length); data = the tensor's bytes"""
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        self.tensors.append((name, ggml_type, tuple(int(x) for x in ne), raw))

    def write(self, path) -> None:
        head = bytearray()
        head += GGUF_MAGIC + struct.pack("<IQQ", GGUF_VERSION, len(self.tensors), len(self.kv))
        for key, vtype, value in self.kv:
            head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
        offsets = []
        off = 0
        for name, gtype, ne, raw in self.tensors:
            offsets.append(off)
            head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
            head += struct.pack("<IQ", gtype, off)
            off = (off + len(raw) + self.alignment - 1) // self.alignment * self.alignment
        pad = (-len(head)) % self.alignment
        with open(path, "wb") as f:
            f.write(head)
            f.write(b"\0" * pad)
            for (name, gtype, ne, raw), o in zip(self.tensors, offsets):
                f.write(raw)
                f.write(b"\0" * ((-len(raw)) % self.alignment))


def export_qwen_pack(weights, path, with_output: bool = False, extra_kv: dict | None = None,
                     alignment: int = 32) -> Path:
    """Write `weights` (openasr_amd.decoders.QwenWeights) as a qwen3-asr pack.
    with_output: also write output.weight (a copy of the tied embedding)."""
    from . import decoders as D

    c = weights.cfg
    w = GGUFWriter(alignment)
    w.add("general.architecture", STR, "qwen3-asr")
    w.add("openasr.package.version", STR, "1")
    w.add("openasr.model.family", STR, "qwen3-asr")
    w.add("openasr.model.architecture", STR, "qwen3-asr")
    for key, val in (("n_layers", c.n_layers), ("d_model", c.d_model), ("n_heads", c.n_head),
                     ("n_kv_heads", c.n_kv_head), ("head_dim", c.head_dim), ("vocab_size", c.vocab)):
        w.add(f"qwen3-asr.llm.{key}", U32, val)
    w.add("qwen3-asr.llm.max_pos", U32, 4096)
    if c.rope_theta != 1e6:
        w.add("qwen3-asr.llm.rope_theta", F32, c.rope_theta)
    for key, (vtype, val) in (extra_kv or {}).items():
        w.add(key, vtype, val)
    wt = c.wtype
    q_w, kv_w = c.n_head * c.head_dim, c.n_kv_head * c.head_dim
    emb = weights.array(-1, D.TOKEN_EMBD)
    w.add_tensor("token_embd.weight", wt, (c.d_model, c.vocab), emb)
    w.add_tensor("output_norm.weight", 0, (c.d_model,), weights.array(-1, D.OUTPUT_NORM))
    if with_output:
        w.add_tensor("output.weight", wt, (c.d_model, c.vocab), emb)
    for layer in range(c.n_layers):
        p = f"blk.{layer}."
        qkv = weights.array(layer, D.QKV)
        row = len(qkv) // (q_w + 2 * kv_w)
        w.add_tensor(p + "attn_norm.weight", 0, (c.d_model,), weights.array(layer, D.ATTN_NORM))
        w.add_tensor(p + "attn_q.weight", wt, (c.d_model, q_w), qkv[:q_w * row])
        w.add_tensor(p + "attn_k.weight", wt, (c.d_model, kv_w), qkv[q_w * row:(q_w + kv_w) * row])
        w.add_tensor(p + "attn_v.weight", wt, (c.d_model, kv_w), qkv[(q_w + kv_w) * row:])
        w.add_tensor(p + "attn_q_norm.weight", 0, (c.head_dim,), weights.array(layer, D.Q_NORM))
        w.add_tensor(p + "attn_k_norm.weight", 0, (c.head_dim,), weights.array(layer, D.K_NORM))
        w.add_tensor(p + "attn_output.weight", wt, (q_w, c.d_model), weights.array(layer, D.O))
        w.add_tensor(p + "ffn_norm.weight", 0, (c.d_model,), weights.array(layer, D.FFN_NORM))
        w.add_tensor(p + "ffn_gate.weight", wt, (c.d_model, c.ffn), weights.array(layer, D.GATE))
        w.add_tensor(p + "ffn_up.weight", wt, (c.d_model, c.ffn), weights.array(layer, D.UP))
        w.add_tensor(p + "ffn_down.weight", wt, (c.ffn, c.d_model), weights.array(layer, D.DOWN))
    w.write(path)
    return Path(path)


# per-layer qwen3-asr audio encoder tensors (models/qwen/tensor_names.rs:23-45):
# (kind in openasr_amd.decoders, name after "audio.blk.N.")
QWEN_AUDIO_LAYER_NAMES = [
    ("QA_ATTN_NORM_W", "attn_norm.weight"), ("QA_ATTN_NORM_B", "attn_norm.bias"), ("QA_Q", "attn_q.weight"),
    ("QA_Q_B", "attn_q.bias"), ("QA_K", "attn_k.weight"), ("QA_K_B", "attn_k.bias"), ("QA_V", "attn_v.weight"),
    ("QA_V_B", "attn_v.bias"), ("QA_O", "attn_out.weight"), ("QA_O_B", "attn_out.bias"),
    ("QA_FFN_NORM_W", "ffn_norm.weight"), ("QA_FFN_NORM_B", "ffn_norm.bias"), ("QA_UP", "ffn_up.weight"),
    ("QA_UP_B", "ffn_up.bias"), ("QA_DOWN", "ffn_down.weight"), ("QA_DOWN_B", "ffn_down.bias"),
]


def export_qwen_audio_pack(weights, path, skip: tuple = (), conv_f16: bool = False, extra_kv: dict | None = None,
                           alignment: int = 32, replace: dict | None = None) -> Path:
    """Write `weights` (openasr_amd.decoders.QwenAudioWeights) as the audio
    encoder half of a qwen3-asr pack (tensor names models/qwen/tensor_names.rs,
    keys arch/hparams.rs:42-52). conv_f16: store the conv kernels as F16 (the
    loader widens them); skip: tensor names left out, replace: name ->
    (ggml type, bytes) stored instead (tests of the loader)."""
    from . import decoders as D

    c = weights.cfg
    w = GGUFWriter(alignment)
    w.add("general.architecture", STR, "qwen3-asr")
    w.add("openasr.package.version", STR, "1")
    for key, val in (("n_mels", c.n_mels), ("audio.n_layers", c.n_layers), ("audio.d_model", c.d_model),
                     ("audio.n_heads", c.n_heads), ("llm.d_model", c.out_dim)):
        w.add(f"qwen3-asr.{key}", U32, val)
    for key, (vtype, val) in (extra_kv or {}).items():
        w.add(key, vtype, val)
    fb = c.n_mels
    for _ in range(3):
        fb = (fb - 1) // 2 + 1
    C_, d = c.conv_channels, c.d_model

    def put(name, gtype, ne, data):
        if name in (replace or {}):
            gtype, data = replace[name]
        if name not in skip:
            w.add_tensor(name, gtype, ne, data)

    for i, (kw, kb) in enumerate(((D.QA_CONV1_W, D.QA_CONV1_B), (D.QA_CONV2_W, D.QA_CONV2_B),
                                  (D.QA_CONV3_W, D.QA_CONV3_B)), start=1):
        ic = 1 if i == 1 else C_
        kern = weights.array(-1, kw)
        if conv_f16:
            put(f"audio.conv.{i}.weight", 1, (3, 3, ic, C_), kern.view(np.float32).astype(np.float16))
        else:
            put(f"audio.conv.{i}.weight", 0, (3, 3, ic, C_), kern)
        put(f"audio.conv.{i}.bias", 0, (C_,), weights.array(-1, kb))
    wt = c.wtype
    put("audio.conv_out.weight", wt, (C_ * fb, d), weights.array(-1, D.QA_CONV_OUT))
    put("audio.conv_out.bias", 0, (d,), weights.array(-1, D.QA_CONV_OUT_B))
    put("audio.ln_post.weight", 0, (d,), weights.array(-1, D.QA_LN_POST_W))
    put("audio.ln_post.bias", 0, (d,), weights.array(-1, D.QA_LN_POST_B))
    put("audio.proj1.weight", wt, (d, d), weights.array(-1, D.QA_PROJ1))
    put("audio.proj1.bias", 0, (d,), weights.array(-1, D.QA_PROJ1_B))
    put("audio.proj2.weight", wt, (d, c.out_dim), weights.array(-1, D.QA_PROJ2))
    put("audio.proj2.bias", 0, (c.out_dim,), weights.array(-1, D.QA_PROJ2_B))
    for layer in range(c.n_layers):
        for kind_name, name in QWEN_AUDIO_LAYER_NAMES:
            kind = getattr(D, kind_name)
            data = weights.array(layer, kind)
            if name.endswith(".bias") or "norm" in name:
                ne = (c.ffn if kind == D.QA_UP_B else d,)
                gtype = 0
            else:
                ne = (c.ffn if kind == D.QA_DOWN else d, c.ffn if kind == D.QA_UP else d)
                gtype = wt
            put(f"audio.blk.{layer}.{name}", gtype, ne, data)
    w.write(path)
    return Path(path)


# per-layer whisper decoder tensors: (kind in openasr_amd.decoders, name after "decoder.layers.N.")
WHISPER_LAYER_NAMES = [
    ("WH_SELF_LN_W", "self_attn_layer_norm.weight"), ("WH_SELF_LN_B", "self_attn_layer_norm.bias"),
    ("WH_SELF_Q", "self_attn.q_proj.weight"), ("WH_SELF_Q_B", "self_attn.q_proj.bias"),
    ("WH_SELF_K", "self_attn.k_proj.weight"), ("WH_SELF_V", "self_attn.v_proj.weight"),
    ("WH_SELF_V_B", "self_attn.v_proj.bias"), ("WH_SELF_O", "self_attn.out_proj.weight"),
    ("WH_SELF_O_B", "self_attn.out_proj.bias"), ("WH_CROSS_LN_W", "encoder_attn_layer_norm.weight"),
    ("WH_CROSS_LN_B", "encoder_attn_layer_norm.bias"), ("WH_CROSS_Q", "cross_attn.q_proj.weight"),
    ("WH_CROSS_Q_B", "cross_attn.q_proj.bias"), ("WH_CROSS_K", "cross_attn.k_proj.weight"),
    ("WH_CROSS_V", "cross_attn.v_proj.weight"), ("WH_CROSS_V_B", "cross_attn.v_proj.bias"),
    ("WH_CROSS_O", "cross_attn.out_proj.weight"), ("WH_CROSS_O_B", "cross_attn.out_proj.bias"),
    ("WH_MLP_LN_W", "final_layer_norm.weight"), ("WH_MLP_LN_B", "final_layer_norm.bias"),
    ("WH_FC1", "fc1.weight"), ("WH_FC1_B", "fc1.bias"), ("WH_FC2", "fc2.weight"), ("WH_FC2_B", "fc2.bias"),
]


def export_whisper_pack(weights, path, extra_kv: dict | None = None, alignment: int = 32, skip: tuple = ()) -> Path:
    """Write `weights` (openasr_amd.decoders.WhisperWeights) as a whisper pack
    (decoder tensors; the encoder's are not part of the decode path). `skip`:
    tensor names left out (tests of the loader's checks)."""
    from . import decoders as D

    c = weights.cfg
    w = GGUFWriter(alignment)
    w.add("general.architecture", STR, "whisper")
    w.add("openasr.package.version", STR, "1")
    for key, val in (("whisper.decoder.block_count", c.n_layers), ("whisper.decoder.embedding_length", c.d_model),
                     ("whisper.decoder.attention.head_count", c.n_head),
                     ("whisper.decoder.context_length", c.max_positions), ("whisper.vocab_size", c.vocab),
                     ("whisper.encoder.context_length", c.n_frames)):
        w.add(key, U32, val)
    for key, (vtype, val) in (extra_kv or {}).items():
        w.add(key, vtype, val)
    Q8_0 = 8
    d = c.d_model

    def put(name, gtype, ne, data):
        if name not in skip:
            w.add_tensor(name, gtype, ne, data)

    put("decoder.token_embedding.weight", Q8_0, (d, c.vocab), weights.array(-1, D.WH_TOKEN_EMBD))
    put("decoder.positional_embedding", 0, (d, c.max_positions), weights.array(-1, D.WH_POS_EMBD))
    put("decoder.layer_norm.weight", 0, (d,), weights.array(-1, D.WH_FINAL_LN_W))
    put("decoder.layer_norm.bias", 0, (d,), weights.array(-1, D.WH_FINAL_LN_B))
    for layer in range(c.n_layers):
        for kind_name, name in WHISPER_LAYER_NAMES:
            kind = getattr(D, kind_name)
            data = weights.array(layer, kind)
            if name.endswith(".bias") or "layer_norm" in name:
                ne = (c.ffn if kind == D.WH_FC1_B else d,)
                gtype = 0
            else:
                ne = (c.ffn if kind == D.WH_FC2 else d, c.ffn if kind == D.WH_FC1 else d)
                gtype = Q8_0
            put(f"decoder.layers.{layer}.{name}", gtype, ne, data)
    w.write(path)
    return Path(path)
