"""The oracle still reproduces the committed fixtures bit for bit
(tests/golden/oracle_fixtures.npz, written by tests/golden/make_golden.py):
a change to the restatement that moves any value fails here first."""

import os

import numpy as np
import pytest

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    assert a.tobytes() == b.tobytes()


def test_quantizers(ref, fx):
    same(ref.quantize_weights(ref.Q8_0, fx["quant_in"]), fx["q8_0_bytes"])
    same(ref.quantize_weights(ref.Q4_K, fx["quant_in"]), fx["q4_K_bytes"])
    same(np.concatenate([ref.quantize_act(ref.Q8_0, r) for r in fx["act_in"]]), fx["act_q8_0_bytes"])
    same(np.concatenate([ref.quantize_act(ref.Q8_K, r) for r in fx["act_in"]]), fx["act_q8_K_bytes"])


@pytest.mark.parametrize("name,typ,m,k", [("mm_q4_K", "Q4_K", 96, 512), ("mm_q8_0", "Q8_0", 64, 256)])
def test_mul_mat(ref, fx, name, typ, m, k):
    same(ref.mul_mat(getattr(ref, typ), fx[name + "_w"], m, k, fx[name + "_x"]), fx[name + "_y"])


def test_row_ops(ref, fx):
    same(ref.rms_norm(fx["norm_in"], 1e-6), fx["rms_norm_out"])
    same(ref.norm(fx["norm_in"], 1e-5), fx["layer_norm_out"])
    same(ref.rope_neox(fx["rope_in"], fx["rope_pos"], 128, 1e6), fx["rope_out"])
    same(ref.soft_max_ext(fx["softmax_in"], fx["softmax_mask"], 0.125), fx["softmax_out"])
    same(ref.silu(fx["act_fn_in"]), fx["silu_out"])
    same(ref.gelu(fx["act_fn_in"]), fx["gelu_out"])


def test_flash_attn(ref, fx):
    for fid, key in ((4, "fa_out"), (5, "fa5_out")):
        out = np.stack([ref.flash_attn(fx["fa_q"][s:s + 1], fx["fa_k"][s], fx["fa_v"][s], fx["fa_mask"][s:s + 1],
                                       0.125, fidelity=fid) for s in range(2)])
        same(out, fx[key])
