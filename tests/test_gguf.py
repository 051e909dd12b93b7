"""The runtime-pack reader (oa_gguf_*, GGUF v2/v3 = the `.oasr` v1 payload)
and the qwen3-asr pack loader, on the CPU: typed metadata and tensor views
read back exactly what the writer put in, malformed files fail closed with a
message (docs/format/OASR_PACKAGE_CONTRACT_V1.md: GGUF magic accepted, the
reserved OASR magic and unknown magics refused), and a pack written from a
decoder's weights loads back byte for byte.
"""

import ctypes as C
import struct

import numpy as np
import pytest

from openasr_amd import decoders as D
from openasr_amd import ggml as G
from openasr_amd import gguf


def open_pack(path):
    err = C.create_string_buffer(512)
    g = D.lib().oa_gguf_open(str(path).encode(), err, len(err))
    return g, err.value.decode()


def tensor(g, name):
    L = D.lib()
    i = L.oa_gguf_find_tensor(g, name.encode())
    assert i >= 0, name
    t, ne = C.c_int(0), (C.c_int64 * 4)()
    nd = L.oa_gguf_tensor_info(g, i, C.byref(t), ne)
    n = C.c_size_t(0)
    p = L.oa_gguf_tensor_data(g, i, C.byref(n))
    data = np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p)).copy()
    return t.value, list(ne)[:nd], data


@pytest.fixture(scope="module")
def sample(tmp_path_factory):
    rng = np.random.default_rng(9)
    w = gguf.GGUFWriter(alignment=64)
    kv = {"t.u8": (gguf.U8, 200), "t.i8": (gguf.I8, -5), "t.u16": (gguf.U16, 65000), "t.i16": (gguf.I16, -300),
          "t.u32": (gguf.U32, 4000000000), "t.i32": (gguf.I32, -70000), "t.u64": (gguf.U64, 1 << 40),
          "t.i64": (gguf.I64, -(1 << 41)), "t.f32": (gguf.F32, 0.25), "t.f64": (gguf.F64, 1e-300),
          "t.bool": (gguf.BOOL, True), "t.str": (gguf.STR, "qwen3-asr ✓"),
          "t.arr": (gguf.ARR, (gguf.U32, [1, 2, 3])), "t.sarr": (gguf.ARR, (gguf.STR, ["a", "bc", ""]))}
    for k, (t, v) in kv.items():
        w.add(k, t, v)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f16 = rng.standard_normal((2, 8)).astype(np.float16)
    q8 = G.quantize(G.Q8_0, rng.standard_normal((4, 64)).astype(np.float32))
    q4 = G.quantize(G.Q4_K, rng.standard_normal((3, 256)).astype(np.float32))
    tensors = {"a.f32": (0, (5, 3), f32), "b.f16": (1, (8, 2), f16), "c.q8": (G.Q8_0, (64, 4), q8),
               "d.q4": (G.Q4_K, (256, 3), q4)}
    for name, (t, ne, data) in tensors.items():
        w.add_tensor(name, t, ne, data)
    path = tmp_path_factory.mktemp("gguf") / "sample.gguf"
    w.write(path)
    return path, kv, tensors


def test_reader_reads_back_metadata_and_tensors(sample):
    path, kv, tensors = sample
    L = D.lib()
    g, err = open_pack(path)
    assert g, err
    try:
        assert L.oa_gguf_version(g) == 3 and L.oa_gguf_alignment(g) == 64
        assert L.oa_gguf_n_tensors(g) == 4 and L.oa_gguf_n_kv(g) == len(kv) + 1  # + general.alignment
        v = C.c_int64(0)
        for k in ("t.u8", "t.i8", "t.u16", "t.i16", "t.u32", "t.i32", "t.u64", "t.i64"):
            assert L.oa_gguf_get_i64(g, k.encode(), C.byref(v)) and v.value == kv[k][1], k
        f = C.c_double(0)
        assert L.oa_gguf_get_f64(g, b"t.f32", C.byref(f)) and f.value == 0.25
        assert L.oa_gguf_get_f64(g, b"t.f64", C.byref(f)) and f.value == 1e-300
        assert L.oa_gguf_get_str(g, b"t.str").decode() == "qwen3-asr ✓"
        assert L.oa_gguf_kv_type(g, b"t.arr") == gguf.ARR and L.oa_gguf_kv_type(g, b"t.bool") == gguf.BOOL
        assert L.oa_gguf_kv_type(g, b"absent") == -1 and not L.oa_gguf_get_str(g, b"t.u8")
        assert not L.oa_gguf_get_i64(g, b"t.str", C.byref(v))
        for name, (t, ne, data) in tensors.items():
            tt, nn, got = tensor(g, name)
            assert tt == t and nn == list(ne) and np.array_equal(got, np.frombuffer(data.tobytes(), np.uint8))
        assert L.oa_gguf_find_tensor(g, b"missing") == -1
    finally:
        L.oa_gguf_close(g)


def corrupt(path, tmp_path, name, fn):
    raw = bytearray(path.read_bytes())
    out = tmp_path / name
    out.write_bytes(bytes(fn(raw)))
    return out


def header_len(raw):
    """byte offset where the tensor infos end (recomputed by walking the header)"""
    pos = 24
    n_t, n_kv = struct.unpack_from("<QQ", raw, 8)

    def s(p):
        n = struct.unpack_from("<Q", raw, p)[0]
        return p + 8 + n
    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
    for _ in range(n_kv):
        pos = s(pos)
        t = struct.unpack_from("<I", raw, pos)[0]
        pos += 4
        if t == 8:
            pos = s(pos)
        elif t == 9:
            et, n = struct.unpack_from("<IQ", raw, pos)
            pos += 12
            for _ in range(n):
                pos = s(pos) if et == 8 else pos + sizes[et]
        else:
            pos += sizes[t]
    infos = []
    for _ in range(n_t):
        infos.append(pos)  # at the name's length prefix
        pos = s(pos)
        nd = struct.unpack_from("<I", raw, pos)[0]
        pos += 4 + 8 * nd + 4 + 8
    return pos, infos


@pytest.mark.parametrize("case", ["oasr_magic", "unknown_magic", "version1", "truncated_kv", "truncated_info",
                                  "truncated_data", "misaligned", "out_of_file", "dup_tensor", "bad_alignment",
                                  "five_dims", "huge_counts"])
def test_reader_fails_closed(sample, tmp_path, case):
    path = sample[0]
    raw0 = path.read_bytes()
    end, infos = header_len(raw0)

    def edit(raw):
        if case == "oasr_magic":
            raw[0:4] = b"OASR"
        elif case == "unknown_magic":
            raw[0:4] = b"GGML"
        elif case == "version1":
            raw[4:8] = struct.pack("<I", 1)
        elif case == "truncated_kv":
            del raw[60:]
        elif case == "truncated_info":
            del raw[end - 6:]
        elif case == "truncated_data":
            del raw[len(raw) - 100:]
        elif case in ("misaligned", "out_of_file"):
            p = infos[1]
            n = struct.unpack_from("<Q", raw, p)[0]
            nd = struct.unpack_from("<I", raw, p + 8 + n)[0]
            off_at = p + 8 + n + 4 + 8 * nd + 4
            struct.pack_into("<Q", raw, off_at, 8 if case == "misaligned" else 1 << 30)
        elif case == "dup_tensor":
            p0, p1 = infos[0], infos[1]
            n0 = struct.unpack_from("<Q", raw, p0)[0]
            n1 = struct.unpack_from("<Q", raw, p1)[0]
            assert n0 == n1  # both names are 5 bytes
            raw[p1 + 8:p1 + 8 + n1] = raw[p0 + 8:p0 + 8 + n0]
        elif case == "bad_alignment":
            i = raw.find(b"general.alignment")
            struct.pack_into("<I", raw, i + len(b"general.alignment") + 4, 48)
        elif case == "five_dims":
            p = infos[0]
            n = struct.unpack_from("<Q", raw, p)[0]
            struct.pack_into("<I", raw, p + 8 + n, 5)
        elif case == "huge_counts":
            struct.pack_into("<Q", raw, 8, 1 << 60)
        return raw
    bad = corrupt(path, tmp_path, case + ".gguf", edit)
    g, err = open_pack(bad)
    assert not g and err
    if case == "oasr_magic":
        assert "reserved" in err
    if case == "unknown_magic":
        assert "magic" in err


def test_reader_missing_file(tmp_path):
    g, err = open_pack(tmp_path / "nope.oasr")
    assert not g and "cannot open" in err


SHAPE = dict(d_model=256, n_layers=2, n_head=4, n_kv_head=2, head_dim=64, ffn=512, vocab=1000)


@pytest.mark.parametrize("wname", ["q8_0", "q4_K"])
def test_qwen_pack_round_trip(tmp_path, wname):
    wt = G.Q8_0 if wname == "q8_0" else G.Q4_K
    w = D.QwenWeights(wt, seed=5, rope_theta=5e5, **SHAPE)
    path = gguf.export_qwen_pack(w, tmp_path / "tiny.oasr", with_output=True)
    w2 = D.QwenWeights.load_gguf(path)
    for f, _ in D.QwenConfig._fields_:
        if f not in ("seed", "out_wtype"):
            assert getattr(w2.cfg, f) == pytest.approx(getattr(w.cfg, f)), f
    for layer in range(-1, SHAPE["n_layers"]):
        kinds = (D.TOKEN_EMBD, D.OUTPUT_NORM) if layer < 0 else D.LAYER_KINDS
        for k in kinds:
            assert np.array_equal(w.array(layer, k), w2.array(layer, k)), (layer, k)
    # output.weight identical to the embedding: tied
    assert w2.tensor(-1, D.OUTPUT) == (None, 0)
    assert w2.pointer_table()[-1] is None


def test_qwen_pack_separate_output(tmp_path):
    w = D.QwenWeights(G.Q4_K, seed=5, **SHAPE)
    other = D.QwenWeights(G.Q8_0, seed=6, **SHAPE)
    wr = gguf.GGUFWriter()
    path = gguf.export_qwen_pack(w, tmp_path / "a.oasr")
    # rewrite with a distinct Q8_0 output projection
    g, _ = open_pack(path)
    names = [D.lib().oa_gguf_tensor_name(g, i).decode() for i in range(D.lib().oa_gguf_n_tensors(g))]
    for key, t, v in (("general.architecture", gguf.STR, "qwen3-asr"), ("openasr.package.version", gguf.STR, "1")):
        wr.add(key, t, v)
    for key in ("n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "vocab_size"):
        iv = C.c_int64(0)
        D.lib().oa_gguf_get_i64(g, f"qwen3-asr.llm.{key}".encode(), C.byref(iv))
        wr.add(f"qwen3-asr.llm.{key}", gguf.U32, iv.value)
    for n in names:
        t, ne, data = tensor(g, n)
        wr.add_tensor(n, t, tuple(ne), data)
    D.lib().oa_gguf_close(g)
    out = other.array(-1, D.TOKEN_EMBD)
    wr.add_tensor("output.weight", G.Q8_0, (SHAPE["d_model"], SHAPE["vocab"]), out)
    wr.write(tmp_path / "b.oasr")
    w2 = D.QwenWeights.load_gguf(tmp_path / "b.oasr")
    assert w2.cfg.out_wtype == G.Q8_0
    assert np.array_equal(w2.array(-1, D.OUTPUT), out)
    assert w2.pointer_table()[-1] is not None


@pytest.mark.parametrize("case,needle", [
    ("missing_tensor", "missing tensor blk.1.ffn_up.weight"),
    ("missing_key", "qwen3-asr.llm.head_dim"),
    ("wrong_arch", "not qwen3-asr"),
    ("bad_version", "openasr.package.version"),
])
def test_qwen_pack_errors(tmp_path, case, needle):
    w = D.QwenWeights(G.Q8_0, seed=5, **SHAPE)
    path = gguf.export_qwen_pack(w, tmp_path / "ok.oasr")
    g, _ = open_pack(path)
    L = D.lib()
    wr = gguf.GGUFWriter()
    wr.add("general.architecture", gguf.STR, "whisper" if case == "wrong_arch" else "qwen3-asr")
    wr.add("openasr.package.version", gguf.STR, "2" if case == "bad_version" else "1")
    for key in ("n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "vocab_size"):
        if case == "missing_key" and key == "head_dim":
            continue
        iv = C.c_int64(0)
        L.oa_gguf_get_i64(g, f"qwen3-asr.llm.{key}".encode(), C.byref(iv))
        wr.add(f"qwen3-asr.llm.{key}", gguf.U32, iv.value)
    for i in range(L.oa_gguf_n_tensors(g)):
        n = L.oa_gguf_tensor_name(g, i).decode()
        if case == "missing_tensor" and n == "blk.1.ffn_up.weight":
            continue
        t, ne, data = tensor(g, n)
        wr.add_tensor(n, t, tuple(ne), data)
    L.oa_gguf_close(g)
    wr.write(tmp_path / "bad.oasr")
    with pytest.raises(ValueError, match=needle):
        D.QwenWeights.load_gguf(tmp_path / "bad.oasr")


WH_SHAPE = dict(d_model=64, n_layers=2, n_head=2, ffn=128, vocab=96, max_positions=16, n_frames=12)


def test_whisper_pack_round_trip(tmp_path):
    w = D.WhisperWeights(seed=7, **WH_SHAPE)
    path = gguf.export_whisper_pack(w, tmp_path / "wh.oasr")
    w2 = D.WhisperWeights.load_gguf(path)
    for f, _ in D.WhisperConfig._fields_:
        if f != "seed":
            assert getattr(w2.cfg, f) == pytest.approx(getattr(w.cfg, f)), f
    for layer in range(WH_SHAPE["n_layers"]):
        for k in range(D.WH_LAYER_KINDS):
            assert np.array_equal(w.array(layer, k), w2.array(layer, k)), (layer, k)
    for k in (D.WH_TOKEN_EMBD, D.WH_POS_EMBD, D.WH_FINAL_LN_W, D.WH_FINAL_LN_B):
        assert np.array_equal(w.array(-1, k), w2.array(-1, k)), k
    w2.free()
    w.free()


@pytest.mark.parametrize("case,needle", [
    ("missing_tensor", "missing tensor decoder.layers.1.cross_attn.v_proj.bias"),
    ("missing_key", "whisper.encoder.context_length"),
    ("wrong_arch", "not whisper"),
    ("wrong_type", "decoder.layers.0.fc1.weight has unsupported type"),
])
def test_whisper_pack_errors(tmp_path, case, needle):
    w = D.WhisperWeights(seed=7, **WH_SHAPE)
    path = gguf.export_whisper_pack(w, tmp_path / "ok.oasr")
    g, _ = open_pack(path)
    L = D.lib()
    wr = gguf.GGUFWriter()
    wr.add("general.architecture", gguf.STR, "qwen3-asr" if case == "wrong_arch" else "whisper")
    for key in ("whisper.decoder.block_count", "whisper.decoder.embedding_length", "whisper.decoder.attention.head_count",
                "whisper.decoder.context_length", "whisper.vocab_size", "whisper.encoder.context_length"):
        if case == "missing_key" and key == "whisper.encoder.context_length":
            continue
        iv = C.c_int64(0)
        L.oa_gguf_get_i64(g, key.encode(), C.byref(iv))
        wr.add(key, gguf.U32, iv.value)
    for i in range(L.oa_gguf_n_tensors(g)):
        n = L.oa_gguf_tensor_name(g, i).decode()
        if case == "missing_tensor" and n == "decoder.layers.1.cross_attn.v_proj.bias":
            continue
        t, ne, data = tensor(g, n)
        if case == "wrong_type" and n == "decoder.layers.0.fc1.weight":
            t, data = G.F32, np.zeros(int(np.prod(ne)), np.float32)
        wr.add_tensor(n, t, tuple(ne), data)
    L.oa_gguf_close(g)
    wr.write(tmp_path / "bad.oasr")
    with pytest.raises(ValueError, match=needle):
        D.WhisperWeights.load_gguf(tmp_path / "bad.oasr")
    w.free()
