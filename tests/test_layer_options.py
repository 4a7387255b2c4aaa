"""Host-side options of the sparse global-attention layer (no GPU needed)."""
import pytest
import torch

from geoweave_amd import dsa_layer


@pytest.mark.parametrize("text,want", [
    ("fp16", torch.float16), ("float16", torch.float16), ("half", torch.float16), ("F16", torch.float16),
    (" bfloat16 ", torch.bfloat16), ("bf16", torch.bfloat16),
    ("", None), ("none", None), (None, None),
    ("int8", None),  # the reference's _parse_dtype returns None for any other spelling
])
def test_score_dtype_spellings_follow_the_reference(text, want):
    # reference: DSAAttention._parse_dtype, dsa_attention.py:503-518
    assert dsa_layer.parse_score_dtype(text) == want


def test_score_dtype_accepts_torch_dtypes():
    assert dsa_layer.parse_score_dtype(torch.float16) == torch.float16
    for fp32 in ("fp32", "float32", "f32", torch.float32):
        assert dsa_layer.parse_score_dtype(fp32) == torch.float32
    for bad in (torch.float64, torch.int8):
        with pytest.raises(TypeError):
            dsa_layer.parse_score_dtype(bad)
    with pytest.raises(TypeError):
        dsa_layer.parse_score_dtype(16)


def test_float32_score_dtype_casts_the_attention_to_bfloat16():
    # dsa_attention.py:4943-4948 casts q/k/v to the score dtype, :5296-5300 casts fp32 q/k/v
    # to bf16 before the sparse kernel; indexer.py:321-326 casts the indexer q/k/w.
    m = dsa_layer.SparseGlobalAttention(dim=128, num_heads=2, topk=8, score_dtype="float32")
    t = torch.zeros(2, dtype=torch.float16)
    out = m._to_score_dtype(torch.float16, t, t, t, t, t, t)
    assert [x.dtype for x in out] == [torch.bfloat16] * 3 + [torch.float32] * 3


def test_layer_keeps_the_score_dtype():
    m = dsa_layer.SparseGlobalAttention(dim=128, num_heads=2, topk=8, score_dtype="float16")
    assert m.score_dtype == torch.float16
    assert dsa_layer.SparseGlobalAttention(dim=128, num_heads=2, topk=8).score_dtype is None


def test_pi3_settings():
    # pi3_training.py:163-167 (pos_type), :253-263 (qkv_bias, qk_norm), pi3.json (score_dtype)
    assert dsa_layer.rope_base_from_pos_type("rope100") == 100.0
    assert dsa_layer.rope_base_from_pos_type("rope37.5") == 37.5
    assert dsa_layer.rope_base_from_pos_type("none") is None
    m = dsa_layer.pi3_global_attention(dim=256, num_heads=4, topk=64)
    assert m.qkv.bias is not None and isinstance(m.q_norm, torch.nn.LayerNorm)
    assert m.rope_base == 100.0 and m.score_dtype == torch.float16


def test_grid_positions_match_the_oracle_restatement():
    from oracle import layer_glue as olg

    got = dsa_layer.grid_positions(3, 37, 37)
    want = olg.pi3_positions(3, 37, 37)
    assert got.dtype == torch.int32 and torch.equal(got.long(), want)
