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


def test_score_dtype_accepts_torch_dtypes_and_refuses_fp32():
    assert dsa_layer.parse_score_dtype(torch.float16) == torch.float16
    for bad in ("fp32", "float32", torch.float32):
        with pytest.raises(TypeError):
            dsa_layer.parse_score_dtype(bad)
    with pytest.raises(TypeError):
        dsa_layer.parse_score_dtype(16)


def test_layer_keeps_the_score_dtype():
    m = dsa_layer.SparseGlobalAttention(dim=128, num_heads=2, topk=8, score_dtype="float16")
    assert m.score_dtype == torch.float16
    assert dsa_layer.SparseGlobalAttention(dim=128, num_heads=2, topk=8).score_dtype is None
