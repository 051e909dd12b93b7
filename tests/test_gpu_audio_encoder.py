"""The Qwen3-ASR audio encoder graph (the decoder's prefix producer,
models/qwen/audio_encoder.rs) on the MI355X backend against the numpy
restatement in oracle/audio_encoder.py on the same synthesised weights and
seeded mel features.

The encoder is a float path (f32 conv stem, f32 / f16 / Q8_0 projections on
the matrix-core GEMM or the quantized tile GEMM, flash attention over f16
K / V), with the reference rounding operands as the device and ggml do, so
that what remains is the order of float sums. The bar is the op tolerance,
2e-3 of the largest output, for f32 and f16 projections. With Q8_0
projections every activation is requantized to int8 per 32-element block:
an order-of-sum difference that moves an activation across a rounding
boundary moves it by a whole quantization step, and the stack carries that
on. The reference run twice with two summation orders (f64 and f32 BLAS)
already differs by up to ~1e-2 of the largest output there, so the Q8_0 bar
is 2e-2.
"""

import numpy as np
import pytest

from openasr_amd import decoders as D
from openasr_amd import ggml as g

SMALL = dict(n_mels=32, conv_channels=32, d_model=256, n_heads=4, n_layers=2, ffn=512, out_dim=96)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def mel_input(n_mels, n_frames, seed):
    return np.random.default_rng(seed).standard_normal((n_mels, n_frames)).astype(np.float32)


def test_token_count_is_13_per_started_chunk():
    """qwen3_audio_token_count_for_mel_frames (audio_encoder.rs:859-867): each
    100-frame chunk (a partial tail padded) passes three stride-2 convs,
    100 -> 50 -> 25 -> 13 rows"""
    from oracle import audio_encoder as RA
    for n, want in ((0, 0), (1, 13), (100, 13), (101, 26), (250, 39), (3000, 390)):
        assert D.qwen_audio_token_count(n) == want == RA.token_count(n), n


def test_weights_refuse_shapes_their_type_cannot_hold():
    with pytest.raises(ValueError):
        D.QwenAudioWeights(g.Q8_0, **dict(SMALL, ffn=500))  # Q8_0 needs K % 32 == 0
    w = D.QwenAudioWeights(g.F16, **SMALL)
    assert w.array(0, D.QA_Q).size == 256 * 256 * 2
    assert w.array(-1, D.QA_CONV2_W).size == 32 * 32 * 9 * 4
    assert w.array(-1, D.QA_CONV_OUT).size == 256 * 32 * 4 * 2  # 32 mel bins -> 4 after the stem
    w.free()


@pytest.mark.parametrize("wname", ["f16", "q8_0"])
def test_runtime_pack_reads_back_tensor_for_tensor(tmp_path, wname):
    """an audio encoder written into a qwen3-asr pack (f16 conv kernels, as
    an fp16 pack stores them) loads back with the same configuration and
    every tensor's bytes (the kernels widened back to the same f32 values)"""
    from openasr_amd import gguf
    wt = g.F16 if wname == "f16" else g.Q8_0
    w = D.QwenAudioWeights(wt, seed=9, **SMALL)
    path = gguf.export_qwen_audio_pack(w, tmp_path / "enc.oasr", conv_f16=True)
    r = D.QwenAudioWeights.load_gguf(path)
    for f in ("n_mels", "conv_channels", "d_model", "n_heads", "n_layers", "ffn", "out_dim", "wtype"):
        assert getattr(r.cfg, f) == getattr(w.cfg, f), f
    for kind in range(D.QA_CONV1_W, D.QA_INV_TIMESCALES + 1):
        a, b = w.array(-1, kind), r.array(-1, kind)
        if kind in (D.QA_CONV1_W, D.QA_CONV2_W, D.QA_CONV3_W):
            a = a.view(np.float32).astype(np.float16).astype(np.float32).view(np.uint8)
        assert np.array_equal(a, b), kind
    for layer in range(SMALL["n_layers"]):
        for kind in range(D.QA_LAYER_KINDS):
            assert np.array_equal(w.array(layer, kind), r.array(layer, kind)), (layer, kind)
    r.free()
    w.free()


@pytest.mark.parametrize("skip,msg", [
    (("audio.blk.1.attn_k.bias",), "missing tensor audio.blk.1.attn_k.bias"),
    (("audio.conv.2.weight",), "missing tensor audio.conv.2.weight"),
    (("audio.ln_post.weight",), "missing tensor audio.ln_post.weight"),
])
def test_runtime_pack_refuses_a_missing_tensor(tmp_path, skip, msg):
    from openasr_amd import gguf
    w = D.QwenAudioWeights(g.F16, seed=9, **SMALL)
    path = gguf.export_qwen_audio_pack(w, tmp_path / "enc.oasr", skip=skip)
    with pytest.raises(ValueError, match=msg):
        D.QwenAudioWeights.load_gguf(path)
    w.free()


def test_runtime_pack_refuses_mixed_projection_types(tmp_path):
    """the encoder's projections share one storage type (all F16, or all
    Q8_0 under the acoustic encoder's floor): an F16 pack with one Q8_0
    matrix is refused by name"""
    from openasr_amd import gguf
    w16 = D.QwenAudioWeights(g.F16, seed=9, **SMALL)
    w8 = D.QwenAudioWeights(g.Q8_0, seed=9, **SMALL)
    path = gguf.export_qwen_audio_pack(w16, tmp_path / "enc.oasr",
                                       replace={"audio.proj1.weight": (g.Q8_0, w8.array(-1, D.QA_PROJ1))})
    with pytest.raises(ValueError, match="audio.proj1.weight is q8_0, the encoder's projections are f16"):
        D.QwenAudioWeights.load_gguf(path)
    w16.free()
    w8.free()


@pytest.mark.gpu
@pytest.mark.parametrize("wname", ["f32", "f16", "q8_0"])
def test_audio_encoder_matches_reference(gpu, wname):
    """three mel chunks (the last one partial) through the whole encoder,
    then a second input of the same chunk count (the graph replayed) and one
    of another (rebuilt)"""
    from oracle import audio_encoder as RA
    wt = {"f32": g.F32, "f16": g.F16, "q8_0": g.Q8_0}[wname]
    print(f"qwen audio encoder {wname}", flush=True)
    w = D.QwenAudioWeights(wt, seed=77, **SMALL)
    enc = D.QwenAudioEncoder(w, gpu.backend)
    enc.set_flash_attention_precision(g.GGML_PREC_F32)  # the exact attention: the projections' bars
    for n_frames, seed in ((250, 1), (270, 2), (100, 3)):
        mel = mel_input(SMALL["n_mels"], n_frames, seed)
        got, ms = enc.encode(mel)
        want = RA.encode(w, mel)
        err = rel_err(got, want)
        spread = rel_err(RA.encode(w, mel, sums="f32"), want)
        print(f"  frames {n_frames}: rows {got.shape[0]}, {ms:.2f} ms, rel err {err:.2e} "
              f"(reference f32 vs f64 sums {spread:.2e})", flush=True)
        assert got.shape == want.shape == (D.qwen_audio_token_count(n_frames), SMALL["out_dim"])
        # each projection type is held to its own precision: the f32 path
        # measures ~1e-6 (an f32 path that rounded an operand to f16 would
        # show ~3e-4), f16 ~3e-4, and Q8_0 moves by whole activation
        # quantization steps where a sum lands near an int8 rounding boundary
        assert err < {"f32": 1e-5, "f16": 2e-3, "q8_0": 2e-2}[wname]
    enc.free()
    w.free()


@pytest.mark.gpu
@pytest.mark.parametrize("wname", ["f32", "f16", "q8_0"])
def test_full_size_audio_encoder_matches_reference(gpu, wname):
    """the Qwen3-ASR-0.6B-shaped encoder the bench times (18 layers of 896,
    14 heads, FFN 3584, 128 mel bins, 480 conv channels, 1024 outputs) over
    three chunks, the last one partial, against the checker (pinned against
    an independent textbook encoder in tests/test_oracle_audio_encoder.py),
    each projection type to its bar"""
    from oracle import audio_encoder as RA
    wt = {"f32": g.F32, "f16": g.F16, "q8_0": g.Q8_0}[wname]
    print(f"full-size qwen audio encoder {wname}", flush=True)
    shape = D.QWEN3_06B_AUDIO
    w = D.QwenAudioWeights(wt, seed=21, **shape)
    enc = D.QwenAudioEncoder(w, gpu.backend)
    enc.set_flash_attention_precision(g.GGML_PREC_F32)
    mel = mel_input(shape["n_mels"], 250, 8)
    got, ms = enc.encode(mel)
    want = RA.encode(w, mel)
    err = rel_err(got, want)
    print(f"  rows {got.shape[0]}, {ms:.2f} ms, rel err {err:.2e}", flush=True)
    assert got.shape == want.shape == (39, shape["out_dim"])
    if wname == "q8_0":
        # 18 layers of int8 requantization: the checker against itself with
        # f32 BLAS sums in place of f64 sets the scale of an order-of-sum
        # difference; the device stays within twice that (and within 5e-2)
        spread = rel_err(RA.encode(w, mel, sums="f32"), want)
        print(f"  checker f32 vs f64 sums: {spread:.2e}", flush=True)
        assert err < min(5e-2, max(2e-2, 2 * spread))
    else:
        # an f32 path that rounded an operand to f16 would show ~5e-4
        assert err < {"f32": 5e-5, "f16": 2e-3}[wname]
    enc.free()
    w.free()


@pytest.mark.gpu
@pytest.mark.parametrize("size", ["small", "full"])
def test_audio_encoder_default_precision(gpu, size):
    """the encoder as the reference builds it (flash attention at
    GGML_PREC_DEFAULT, cpu_graph.rs:4120-4142): the attention on the matrix
    cores (P rounded to f16 for P V) with f32 projections, within the op
    tolerance 2e-3 of the checker; the exact contract on the same encoder
    moves by less"""
    from oracle import audio_encoder as RA
    shape = SMALL if size == "small" else D.QWEN3_06B_AUDIO
    print(f"qwen audio encoder {size}, f32 projections, default-precision attention", flush=True)
    w = D.QwenAudioWeights(g.F32, seed=23, **shape)
    enc = D.QwenAudioEncoder(w, gpu.backend)
    mel = mel_input(shape["n_mels"], 250, 9)
    want = RA.encode(w, mel)
    got, ms = enc.encode(mel)
    err = rel_err(got, want)
    enc.set_flash_attention_precision(g.GGML_PREC_F32)
    exact, ms32 = enc.encode(mel)
    err32 = rel_err(exact, want)
    print(f"  default {ms:.2f} ms, rel err {err:.2e}; exact attention {ms32:.2f} ms, rel err {err32:.2e}",
          flush=True)
    assert err < 2e-3 and err32 <= err
    enc.free()
    w.free()


@pytest.mark.gpu
def test_runtime_pack_encodes_like_synthesized(gpu, tmp_path):
    """the encoder bound from a qwen3-asr pack (f32 conv kernels, F16
    projections) gives the same bits as the synthesised weights it was
    written from"""
    from openasr_amd import gguf
    w = D.QwenAudioWeights(g.F16, seed=13, **SMALL)
    path = gguf.export_qwen_audio_pack(w, tmp_path / "enc.oasr")
    r = D.QwenAudioWeights.load_gguf(path)
    mel = mel_input(SMALL["n_mels"], 230, 4)
    a = D.QwenAudioEncoder(w, gpu.backend)
    b = D.QwenAudioEncoder(r, gpu.backend)
    ya, _ = a.encode(mel)
    yb, _ = b.encode(mel)
    assert np.array_equal(ya, yb)
    a.free()
    b.free()
    r.free()
    w.free()
