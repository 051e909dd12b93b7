"""Pins the oracle's decoder compositions (oracle/ref_decoder.c): which
tensor feeds which op, in what order, with which residual, over tiny seeded
models whose weights are built here (random norm weights, so a swapped norm
shows). The per-op arithmetic is pinned in test_oracle.py; these pin the
wiring, by three independent routes:

  1. batched == serial: one batched decode step over ragged positions equals
     the per-sequence forward bit for bit (nn/decoder.rs:3412-3520);
  2. identity reductions, bit-exact against the pinned primitives: with the
     attention and MLP output projections zeroed every layer passes the
     residual stream through, so the logits are the head applied to the
     final norm of the embedding; at position 0 the attention returns the
     value row of the query's KV head;
  3. an f64 numpy restatement of the Qwen3 llm_layer (nn/decoder.rs:1850-2145,
     nn/ffn.rs:64-91, llm_transformer.rs:2096-2115) and of the Whisper
     decoder layer (models/whisper/ggml_decoder_graph.rs:4557-5392) with
     textbook attention, agreeing within 2e-3 of the logit range (the seeds
     here agree to ~1e-7: the restatement keeps ggml's activation
     quantization, f16 KV rows and f16 GELU table); each planted
     composition mistake (residual from the normed input, k_norm on q, the
     wrong GQA head, SiLU on the up branch, GPT-J rope pairs, the cross
     attention reading the self cache, ...) moves the restatement outside
     that bound (by 15-80% of the logit range), so the same mistake in the
     oracle would fail.

Host code only, no GPU.
"""

from types import SimpleNamespace

import numpy as np
import pytest

TOL = 2e-3  # of the largest |logit|


def f32(x):
    return np.asarray(x, np.float32)


def f16_round(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def addr(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------ Qwen3 --

class TinyQwen:
    """A Qwen3-shaped decoder built from seeded numpy arrays: N(0, 1/k)
    matrices quantized by the pinned quantizers, U(0.5, 1.5) norm weights.
    Head dim 64, 4 query heads over 2 KV heads (GQA 2)."""

    def __init__(self, ref, wtype, seed, n_layers=2, tied=True, d=256, hq=4, hkv=2, hd=64, ffn=512, vocab=300,
                 theta=1e4):
        self.ref = ref
        rng = np.random.default_rng(seed)
        self.cfg = SimpleNamespace(d_model=d, n_layers=n_layers, n_head=hq, n_kv_head=hkv, head_dim=hd, ffn=ffn,
                                   vocab=vocab, wtype=wtype, rope_theta=theta, rms_eps=1e-6, out_wtype=ref.Q8_0)
        q_w, kv_w = hq * hd, hkv * hd

        def mat(rows, k, typ=wtype, scale=None):
            x = rng.standard_normal((rows, k)) * (scale if scale is not None else k ** -0.5)
            return ref.quantize_weights(typ, f32(x))

        vec = lambda n: f32(rng.uniform(0.5, 1.5, n))  # noqa: E731
        self.embd = mat(vocab, d, scale=1.0)
        self.out_norm = vec(d)
        self.layers = []
        for _ in range(n_layers):
            self.layers.append(dict(attn_norm=vec(d), qkv=mat(q_w + 2 * kv_w, d), q_norm=vec(hd), k_norm=vec(hd),
                                    o=mat(d, q_w), ffn_norm=vec(d), gate=mat(ffn, d), up=mat(ffn, d),
                                    down=mat(d, ffn)))
        self.out = None if tied else mat(vocab, d, typ=ref.Q8_0)

    KINDS = ("attn_norm", "qkv", "q_norm", "k_norm", "o", "ffn_norm", "gate", "up", "down")

    def table(self):
        t = [addr(self.embd), addr(self.out_norm)]
        for L in self.layers:
            t += [addr(L[k]) for k in self.KINDS]
        return t + [addr(self.out)]

    def head(self):
        return (self.ref.Q8_0, self.out) if self.out is not None else (self.cfg.wtype, self.embd)

    def embed(self, tokens):
        c = self.cfg
        rs = self.ref.row_size(c.wtype, c.d_model)
        return np.stack([self.ref.dequantize(c.wtype, self.embd[t * rs:(t + 1) * rs], c.d_model) for t in tokens])

    def oracle(self, max_pos=16):
        return self.ref.QwenRef(self.cfg, self.table(), max_pos, fa_fidelity=5)


def act_type(ref, wtype):
    return ref.Q8_K if wtype == ref.Q4_K else ref.Q8_0


def mm64(ref, wtype, w, m, k, x):
    """f64 product with ggml's activation quantization: each row of x is
    quantized to the weight's dot type (pinned separately) and the f64 dot is
    taken against the dequantized weight"""
    W = ref.dequantize(wtype, w, m * k).reshape(m, k).astype(np.float64)
    at = act_type(ref, wtype)
    xq = np.stack([ref.dequantize(at, ref.quantize_act(at, f32(r)), k) for r in np.atleast_2d(x)])
    return xq.astype(np.float64) @ W.T


def rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def rope64(x, pos, theta, gptj=False):
    """x [T, H, D]; NeoX pairs (i, i + D/2), or adjacent pairs (2i, 2i+1)"""
    T, H, D = x.shape
    half = D // 2
    inv = theta ** (-np.arange(half) * 2.0 / D)
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    y = x.copy()
    a, b = (x[..., 0::2], x[..., 1::2]) if gptj else (x[..., :half], x[..., half:])
    ra, rb = a * c - b * s, a * s + b * c
    if gptj:
        y[..., 0::2], y[..., 1::2] = ra, rb
    else:
        y[..., :half], y[..., half:] = ra, rb
    return y


def attend64(q, k, v, causal, kv_head):
    """textbook softmax attention; q [T, Hq, D], k/v [S, Hkv, D]; query head h
    reads KV head kv_head(h); position t sees 0..t when causal"""
    T, Hq, D = q.shape
    out = np.zeros_like(q)
    for t in range(T):
        span = t + 1 if causal else k.shape[0]
        for h in range(Hq):
            g = kv_head(h)
            s = k[:span, g] @ q[t, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v[:span, g]
    return out


def silu64(x):
    return x / (1.0 + np.exp(-x))


def qwen64(M, x, bug=None):
    """logits [T, vocab] of every position of the layer-0 input x [T, d]"""
    ref, c = M.ref, M.cfg
    d, hq, hkv, hd, ffn = c.d_model, c.n_head, c.n_kv_head, c.head_dim, c.ffn
    q_w, kv_w = hq * hd, hkv * hd
    T = len(x)
    pos = np.arange(T)
    group = hq // hkv
    kv_head = (lambda h: h % hkv) if bug == "gqa_modulo" else (lambda h: h // group)
    x = np.asarray(x, np.float64)
    for L in M.layers:
        n = rms64(x, L["attn_norm"], c.rms_eps)
        qkv = mm64(ref, c.wtype, L["qkv"], q_w + 2 * kv_w, d, n)
        q = qkv[:, :q_w].reshape(T, hq, hd)
        k = qkv[:, q_w:q_w + kv_w].reshape(T, hkv, hd)
        v = qkv[:, q_w + kv_w:].reshape(T, hkv, hd)
        q = rms64(q, L["k_norm"] if bug == "k_norm_on_q" else L["q_norm"], c.rms_eps)
        k = rms64(k, L["k_norm"], c.rms_eps)
        q = rope64(q, pos, c.rope_theta, gptj=bug == "rope_gptj")
        k = rope64(k, pos, c.rope_theta, gptj=bug == "rope_gptj")
        a = attend64(f16_round(q), f16_round(k), f16_round(v), True, kv_head)
        o = mm64(ref, c.wtype, L["o"], d, q_w, a.reshape(T, q_w))
        x = (n if bug == "residual_from_normed" else x) + o
        n = rms64(x, L["attn_norm"] if bug == "ffn_uses_attn_norm" else L["ffn_norm"], c.rms_eps)
        g = mm64(ref, c.wtype, L["gate"], ffn, d, n)
        u = mm64(ref, c.wtype, L["up"], ffn, d, n)
        h = silu64(u) * g if bug == "silu_on_up" else silu64(g) * u
        x = x + mm64(ref, c.wtype, L["down"], d, ffn, h)
    n = rms64(x, 1.0 if bug == "no_output_norm_weight" else M.out_norm, c.rms_eps)
    ht, hw = M.head()
    return mm64(ref, ht, hw, c.vocab, d, n)


QWEN_BUGS = ("residual_from_normed", "k_norm_on_q", "gqa_modulo", "rope_gptj", "silu_on_up", "ffn_uses_attn_norm",
             "no_output_norm_weight")


def rel_err(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


@pytest.mark.parametrize("wtype_name,tied", [("Q8_0", True), ("Q4_K", True), ("Q4_K", False)])
def test_qwen_batched_step_equals_serial(ref, wtype_name, tied):
    """three sequences prefilled to different lengths, then four batched
    greedy steps: every step's logits and every written cache row equal the
    per-sequence forward's, bit for bit"""
    M = TinyQwen(ref, getattr(ref, wtype_name), seed=11, tied=tied)
    rng = np.random.default_rng(3)
    lens = [1, 4, 7]
    serial = [M.oracle() for _ in lens]
    for r, T in zip(serial, lens):
        r.forward(f32(rng.standard_normal((T, M.cfg.d_model))))
    rb = ref.QwenRefBatch(M.cfg, M.table(), 16, len(lens), fa_fidelity=5)
    for s, r in enumerate(serial):
        for layer in range(M.cfg.n_layers):
            np.copyto(rb.k[s][layer], r.k[layer])
            np.copyto(rb.v[s][layer], r.v[layer])
    rb.pos[:] = lens
    tokens = np.array([5, 17, 250], np.int32)
    for _ in range(4):
        top, logits = rb.step(tokens, want_logits=True)
        for s, r in enumerate(serial):
            t1, lg = r.step(int(tokens[s]))
            assert t1 == top[s]
            assert np.array_equal(lg.view(np.uint32), logits[s].view(np.uint32)), s
        tokens = top
    for s, r in enumerate(serial):
        for layer in range(M.cfg.n_layers):
            assert np.array_equal(rb.k[s][layer], r.k[layer]) and np.array_equal(rb.v[s][layer], r.v[layer])


@pytest.mark.parametrize("wtype_name,tied", [("Q8_0", False), ("Q4_K", True)])
def test_qwen_zeroed_branches_pass_the_residual_stream(ref, wtype_name, tied):
    """o and down projections all zero (zero bytes are zero blocks in both
    formats): the logits at every step are head(rms_norm(embedding) * w_out)
    computed with the pinned primitives, bit for bit"""
    M = TinyQwen(ref, getattr(ref, wtype_name), seed=12, n_layers=3, tied=tied)
    for L in M.layers:
        L["o"][:] = 0
        L["down"][:] = 0
    r = M.oracle()
    ht, hw = M.head()
    for token in (3, 299, 3, 120):
        _, lg = r.step(token)
        x = M.embed([token])
        want = ref.mul_mat(ht, hw, M.cfg.vocab, M.cfg.d_model, ref.rms_norm(x, M.cfg.rms_eps) * M.out_norm)[0]
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32))


def test_qwen_first_position_attends_to_its_own_value_row(ref):
    """at position 0 the only live key is the token's own: each query head's
    attention output is the f16 value row of its KV head (h // 2 with GQA 2),
    so with the MLP zeroed the logits are head(norm(x + W_o v_rows))"""
    M = TinyQwen(ref, ref.Q8_0, seed=13, n_layers=1)
    L = M.layers[0]
    L["down"][:] = 0
    r = M.oracle()
    c = M.cfg
    _, lg = r.step(42)
    v_rows = r.v[0][:, 0, :].view(np.float16).astype(np.float32)  # [hkv, hd]
    assert not np.array_equal(v_rows[0], v_rows[1])
    att = np.concatenate([v_rows[h // (c.n_head // c.n_kv_head)] for h in range(c.n_head)])[None, :]
    x = M.embed([42])
    x1 = x + ref.mul_mat(c.wtype, L["o"], c.d_model, c.n_head * c.head_dim, att)
    ht, hw = M.head()
    want = ref.mul_mat(ht, hw, c.vocab, c.d_model, ref.rms_norm(x1, c.rms_eps) * M.out_norm)[0]
    assert np.array_equal(lg.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wtype_name,tied", [("Q8_0", True), ("Q4_K", False)])
def test_qwen_oracle_matches_f64_restatement(ref, wtype_name, tied):
    """prefill of 3 embedding positions then 4 token steps through 2 layers:
    every step's logits within 2e-3 of the f64 restatement; every planted
    composition mistake lands outside that bound"""
    M = TinyQwen(ref, getattr(ref, wtype_name), seed=14, tied=tied)
    rng = np.random.default_rng(5)
    prefix = f32(rng.standard_normal((3, M.cfg.d_model)))
    r = M.oracle()
    _, lg = r.forward(prefix)
    seq = [prefix]
    got = [lg]
    for token in (7, 77, 177, 277):
        _, lg = r.step(token)
        seq.append(M.embed([token]))
        got.append(lg)
    x = np.concatenate(seq)
    steps = [2, 3, 4, 5, 6]  # the positions whose logits the oracle returned
    want = qwen64(M, x)[steps]
    err = max(rel_err(g, w) for g, w in zip(got, want))
    assert err <= TOL, err
    for bug in QWEN_BUGS:
        planted = qwen64(M, x, bug)[steps]
        e = max(rel_err(g, w) for g, w in zip(got, planted))
        assert e > 5 * TOL, (bug, e)


# ---------------------------------------------------------------- Whisper --

WH_KINDS = ("self_ln_w", "self_ln_b", "self_q", "self_q_b", "self_k", "self_v", "self_v_b", "self_o", "self_o_b",
            "cross_ln_w", "cross_ln_b", "cross_q", "cross_q_b", "cross_k", "cross_v", "cross_v_b", "cross_o",
            "cross_o_b", "mlp_ln_w", "mlp_ln_b", "fc1", "fc1_b", "fc2", "fc2_b")


class TinyWhisper:
    """A Whisper-shaped decoder from seeded numpy arrays (Q8_0 matrices),
    d 128, 2 heads of 64, FFN 256, 16 positions, 40 encoder frames."""

    def __init__(self, ref, seed, n_layers=2, d=128, H=2, ffn=256, vocab=200, max_positions=16, n_frames=40,
                 ffn_act=0):
        self.ref = ref
        rng = np.random.default_rng(seed)
        self.cfg = SimpleNamespace(d_model=d, n_layers=n_layers, n_head=H, ffn=ffn, vocab=vocab,
                                   max_positions=max_positions, n_frames=n_frames, ln_eps=1e-5, ffn_act=ffn_act)

        def mat(rows, k, scale=None):
            x = rng.standard_normal((rows, k)) * (scale if scale is not None else k ** -0.5)
            return ref.quantize_weights(ref.Q8_0, f32(x))

        self.layers = []
        for _ in range(n_layers):
            L = {}
            for kind in WH_KINDS:
                if kind.endswith("_ln_w"):
                    L[kind] = f32(rng.uniform(0.5, 1.5, d))
                elif kind.endswith("_b"):
                    L[kind] = f32(rng.standard_normal(ffn if kind == "fc1_b" else d) * 0.3)
                else:
                    rows = ffn if kind == "fc1" else d
                    L[kind] = mat(rows, ffn if kind == "fc2" else d)
            self.layers.append(L)
        self.tok = mat(vocab, d, scale=1.0)
        self.pos = f32(rng.standard_normal((max_positions, d)) * 0.5)
        self.fin_w = f32(rng.uniform(0.5, 1.5, d))
        self.fin_b = f32(rng.standard_normal(d) * 0.3)

    def table(self):
        t = [addr(L[k]) for L in self.layers for k in WH_KINDS]
        return t + [addr(self.tok), addr(self.pos), addr(self.fin_w), addr(self.fin_b)]

    def embed(self, token, p):
        rs = self.ref.row_size(self.ref.Q8_0, self.cfg.d_model)
        return self.ref.dequantize(self.ref.Q8_0, self.tok[token * rs:(token + 1) * rs], self.cfg.d_model) + self.pos[p]

    def oracle(self, enc):
        r = self.ref.WhisperRef(self.cfg, self.table(), fa_fidelity=5)
        r.set_encoder(enc)
        return r


def ln64(x, w, b, eps):
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def gelu64(x):
    """ggml-cpu's GELU: the tanh form looked up in an f16 table (input and
    output rounded to f16), x past +-10 short-circuited. Without the f16
    rounding the logits move by ~5e-3 of their range on this model."""
    g = lambda t: 0.5 * t * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (t + 0.044715 * t ** 3)))  # noqa: E731
    return np.where(x <= -10, 0.0, np.where(x >= 10, x, f16_round(g(f16_round(x)))))


def act64(act, x):
    """the seq2seq FFN activations (nn/decoder.rs:1125-1138) in f64: GELU
    through ggml's f16 table, RELU, GELU_ERF, SILU"""
    if act == 1:
        return np.maximum(x, 0.0)
    if act == 2:
        from math import erf
        return 0.5 * x * (1.0 + np.vectorize(erf)(x / np.sqrt(2.0)))
    if act == 3:
        return silu64(x)
    return gelu64(x)


def whisper64(M, enc, tokens, bug=None):
    """logits [T, vocab] of the tokens at positions 0..T-1"""
    ref, c = M.ref, M.cfg
    d, H, ffn = c.d_model, c.n_head, c.ffn
    hd = d // H
    T, F = len(tokens), len(enc)
    lin = lambda w, m, k, x, b=None: mm64(ref, ref.Q8_0, w, m, k, x) + (0.0 if b is None else b)  # noqa: E731
    x = np.stack([M.embed(t, p) for p, t in enumerate(tokens)]).astype(np.float64)
    ident = lambda h: h  # noqa: E731
    for L in M.layers:
        lnb = (lambda k: 0.0) if bug == "ln_without_bias" else (lambda k: L[k])
        n = ln64(x, L["self_ln_w"], lnb("self_ln_b"), c.ln_eps)
        q = lin(L["self_q"], d, d, n, L["self_q_b"])
        k = lin(L["self_k"], d, d, n)
        v = lin(L["self_v"], d, d, n, L["self_v_b"])
        sk, sv = f16_round(k).reshape(T, H, hd), f16_round(v).reshape(T, H, hd)
        a = attend64(f16_round(q).reshape(T, H, hd), sk, sv, True, ident)
        o = lin(L["self_o"], d, d, a.reshape(T, d), L["self_o_b"])
        x = (n if bug == "residual_from_normed" else x) + o
        n = ln64(x, L["cross_ln_w"], lnb("cross_ln_b"), c.ln_eps)
        q = lin(L["cross_q"], d, d, n, L["cross_q_b"])
        if bug == "cross_reads_self_cache":
            ck, cv, causal = sk, sv, True
        else:
            ck = f16_round(lin(L["cross_k"], d, d, enc)).reshape(F, H, hd)
            cv = f16_round(lin(L["cross_v"], d, d, enc, L["cross_v_b"])).reshape(F, H, hd)
            causal = False
        a = attend64(f16_round(q).reshape(T, H, hd), ck, cv, causal, ident)
        x = x + lin(L["cross_o"], d, d, a.reshape(T, d), L["cross_o_b"])
        n = ln64(x, L["mlp_ln_w"], lnb("mlp_ln_b"), c.ln_eps)
        h = lin(L["fc1"], ffn, d, n, L["fc1_b"])
        act = getattr(c, "ffn_act", 0)
        if bug == "wrong_activation":
            act = (act + 1) % 4
        h = h if bug == "no_gelu" else act64(act, h)
        x = x + lin(L["fc2"], d, ffn, h, L["fc2_b"])
    n = ln64(x, M.fin_w, 0.0 if bug == "ln_without_bias" else M.fin_b, c.ln_eps)
    return mm64(ref, ref.Q8_0, M.tok, c.vocab, d, n)


WHISPER_BUGS = ("residual_from_normed", "ln_without_bias", "cross_reads_self_cache", "no_gelu", "wrong_activation")


@pytest.mark.parametrize("ffn_act", [0, 1, 2, 3])
def test_whisper_oracle_matches_f64_restatement(ref, ffn_act):
    """the seq2seq block with each FFN activation (0 GELU, 1 RELU, 2 GELU_ERF, 3 SILU)"""
    M = TinyWhisper(ref, seed=21, ffn_act=ffn_act)
    enc = f32(np.random.default_rng(6).standard_normal((M.cfg.n_frames, M.cfg.d_model)))
    r = M.oracle(enc)
    tokens = [3, 150, 150, 9, 77]
    got = [r.step(t)[1] for t in tokens]
    want = whisper64(M, enc, tokens)
    err = max(rel_err(g, w) for g, w in zip(got, want))
    assert err <= TOL, err
    for bug in WHISPER_BUGS:
        planted = whisper64(M, enc, tokens, bug)
        e = max(rel_err(g, w) for g, w in zip(got, planted))
        assert e > 5 * TOL, (bug, e)


def test_whisper_zeroed_branches_pass_the_residual_stream(ref):
    """self-attention output, cross-attention output and fc2 weights and
    biases zeroed: the logits are tok_embd . (LN(tok + pos) * w + b), bit for bit"""
    M = TinyWhisper(ref, seed=22)
    for L in M.layers:
        for k in ("self_o", "self_o_b", "cross_o", "cross_o_b", "fc2", "fc2_b"):
            L[k][:] = 0
    enc = f32(np.random.default_rng(7).standard_normal((M.cfg.n_frames, M.cfg.d_model)))
    r = M.oracle(enc)
    c = M.cfg
    for p, token in enumerate((5, 199, 5)):
        _, lg = r.step(token)
        x = f32(M.embed(token, p))[None, :]
        n = ref.norm(x, c.ln_eps) * M.fin_w + M.fin_b
        want = ref.mul_mat(ref.Q8_0, M.tok, c.vocab, c.d_model, n)[0]
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), p


def test_whisper_first_position_attends_to_its_own_value_row(ref):
    """position 0: the self attention returns the token's own f16 value row
    (bias included) per head; with the cross-attention output and the MLP
    zeroed the logits are head(LN(x + W_o v + b_o)), bit for bit"""
    M = TinyWhisper(ref, seed=23, n_layers=1)
    L = M.layers[0]
    for k in ("cross_o", "cross_o_b", "fc2", "fc2_b"):
        L[k][:] = 0
    enc = f32(np.random.default_rng(8).standard_normal((M.cfg.n_frames, M.cfg.d_model)))
    r = M.oracle(enc)
    c = M.cfg
    _, lg = r.step(31)
    v = r.v[0][0].view(np.float16).astype(np.float32)[None, :]
    x = f32(M.embed(31, 0))[None, :]
    x1 = ref.mul_mat(ref.Q8_0, L["self_o"], c.d_model, c.d_model, v) + L["self_o_b"] + x
    n = ref.norm(x1, c.ln_eps) * M.fin_w + M.fin_b
    want = ref.mul_mat(ref.Q8_0, M.tok, c.vocab, c.d_model, n)[0]
    assert np.array_equal(lg.view(np.uint32), want.view(np.uint32))
