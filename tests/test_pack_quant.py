"""The pack writer's storage policy (oa_classify_quant_tensor_role,
oa_quant_target_write_type) on the known-answer cases of the reference's
own tests (crates/openasr-core/src/models/pack_quant.rs:220-475): the
shapes, rungs, roles and expected ggml types are the reference's; its None
is None here. Host code only, no GPU.
"""

import pytest

from openasr_amd import decoders as D
from openasr_amd import ggml as G

FIRST, LAST = D.AXIS_FIRST, D.AXIS_LAST
DEC, ENC = D.ROLE_TEXT_DECODER_MATRIX, D.ROLE_ACOUSTIC_ENCODER_MATRIX
Q8_0, Q4_K, Q3_K = G.Q8_0, G.Q4_K, D.GGML_Q3_K


def classify(dims, rung, role, axis=FIRST):
    return D.classify_quant_tensor_role(dims, rung, role, axis)


def test_fp16_tier_never_produces_a_block_quant():
    """:220-240"""
    assert classify([256], D.PACK_FP16, DEC) is None
    assert classify([256], D.PACK_FP16, ENC) is None


def test_inventory_projection_only_block_quantizes_rank_two_matrices():
    """:242-268: a decoder-role contract, then a whole-acoustic-pack contract
    (role acoustic encoder, first axis)"""
    assert D.target_write_type([256], D.PACK_Q4_K, DEC) is None
    assert D.target_write_type([256, 4, 3], D.PACK_Q4_K, DEC) is None
    assert D.target_write_type([256, 4], D.PACK_Q4_K, DEC) == Q4_K
    assert D.target_write_type([32, 4], D.PACK_Q4_K, ENC) == Q8_0
    assert D.target_write_type([256, 4], D.PACK_Q4_K, None) is None  # a contract with no acoustic encoder


def test_unaligned_ne0_falls_back_to_fp16_representation():
    """:270-301"""
    assert classify([31], D.PACK_Q8_0, DEC) is None
    assert classify([32], D.PACK_Q8_0, DEC) == Q8_0
    assert classify([31], D.PACK_Q4_K, ENC) is None


@pytest.mark.parametrize("rung,ktype", [(D.PACK_Q4_K, Q4_K), (D.PACK_Q3_K, Q3_K)])
def test_k_quant_requires_256_alignment_else_falls_back_to_q8_0(rung, ktype):
    """:303-345"""
    assert classify([32], rung, DEC) == Q8_0
    assert classify([256], rung, DEC) == ktype


def test_encoder_carries_a_q8_0_floor_below_the_requested_rung():
    """:347-389"""
    assert classify([256], D.PACK_Q4_K, ENC) == Q8_0
    assert classify([256], D.PACK_Q3_K, ENC) == Q8_0
    assert classify([256], D.PACK_Q8_0, ENC) == Q8_0
    assert classify([32], D.PACK_Q4_K, ENC) == Q8_0


def test_precision_critical_matrices_share_the_q8_floor_policy():
    """:391-412"""
    assert classify([256, 5000], D.PACK_Q4_K, D.ROLE_PRECISION_CRITICAL_MATRIX) == Q8_0
    assert classify([256, 256], D.PACK_Q4_K, DEC) == Q4_K


def test_decoder_keeps_the_full_requested_rung():
    """:414-434, and the embedding table and output projection (no floor,
    :161-169)"""
    assert classify([256], D.PACK_Q4_K, DEC) == Q4_K
    assert classify([256], D.PACK_Q3_K, DEC) == Q3_K
    for role in (D.ROLE_EMBEDDING_TABLE, D.ROLE_OUTPUT_PROJECTION):
        assert classify([1024, 151936], D.PACK_Q4_K, role) == Q4_K


def test_semantic_roles_apply_policy_without_tensor_names():
    """:436-465"""
    assert classify([256, 896], D.PACK_Q4_K, ENC) == Q8_0
    assert classify([896, 256], D.PACK_Q4_K, DEC, LAST) == Q4_K
    assert classify([256, 896], D.PACK_Q4_K, D.ROLE_NON_QUANTIZABLE) is None


def test_label_matches_canonical_pack_quant_tags():
    """:467-474"""
    assert [D.PACK_LABELS[r] for r in (D.PACK_FP16, D.PACK_Q8_0, D.PACK_Q3_K, D.PACK_Q4_K)] == \
        ["fp16", "q8_0", "q3_k", "q4_k"]


def test_out_of_range_arguments_are_refused():
    with pytest.raises(ValueError):
        classify([256], 9, DEC)
    with pytest.raises(ValueError):
        classify([256], D.PACK_Q4_K, 17)
    with pytest.raises(ValueError):
        classify([256], D.PACK_Q4_K, DEC, 5)


def test_synthesised_weights_follow_the_policy():
    """a Q4_K decoder whose matrices are not 256-aligned would be stored
    Q8_0 by the writer: the builder refuses it rather than write bytes no
    pack holds"""
    with pytest.raises(ValueError, match="q4_k pack stores it as ggml type 8"):
        D.QwenWeights(G.Q4_K, seed=1, d_model=128, n_layers=1, n_head=2, n_kv_head=1, head_dim=64, ffn=256,
                      vocab=64)
