"""Host-side rules of the indexer drop-in (no GPU needed)."""
import pytest
import torch

from geoweave_amd.custom_indexer import sparse_topk_indexer as sti


def test_view_bias_shape_rules_follow_the_reference():
    # reference: _normalize_view_bias_data, sparse_topk_indexer.py:621-659
    vb = dict(q_view_ids=torch.tensor([0, 1, 1]), s_view_ids=torch.tensor([1, 0, 1, 0]),
              view_bias=torch.tensor([[0.0, 2.0], [1.5, 0.0]]))
    n = sti._normalize_view_bias_data(vb, 2, 3, 4, "cpu", torch.bfloat16)
    assert n["q_view_ids"].shape == (2, 3) and n["q_view_ids"].dtype == torch.long
    assert n["s_view_ids"].shape == (2, 4) and n["s_view_ids"].dtype == torch.long
    assert n["view_bias"].shape == (2, 2, 2) and n["view_bias"].dtype == torch.bfloat16
    assert torch.equal(n["q_view_ids"][1], torch.tensor([0, 1, 1]))
    # a dict missing any key is no view bias
    for key in vb:
        part = {kk: v for kk, v in vb.items() if kk != key}
        assert sti._normalize_view_bias_data(part, 2, 3, 4, "cpu", torch.bfloat16) is None
    assert sti._normalize_view_bias_data(None, 2, 3, 4, "cpu", torch.bfloat16) is None


@pytest.mark.parametrize("bad", [
    dict(q_view_ids=torch.zeros(5, dtype=torch.long)),            # wrong T
    dict(s_view_ids=torch.zeros(2, 3, dtype=torch.long)),         # wrong S
    dict(view_bias=torch.zeros(3, 2, 2)),                         # batch 3 for B = 2
    dict(view_bias=torch.zeros(2, 2, 2, 1)),                      # not [B, Vq, Vs]
])
def test_view_bias_shape_errors(bad):
    vb = dict(q_view_ids=torch.zeros(3, dtype=torch.long), s_view_ids=torch.zeros(4, dtype=torch.long),
              view_bias=torch.zeros(2, 2))
    vb.update(bad)
    with pytest.raises(ValueError):
        sti._normalize_view_bias_data(vb, 2, 3, 4, "cpu", torch.float16)


def test_view_ids_are_range_checked():
    qv = torch.tensor([[0, 1]])
    sv = torch.tensor([[0, 0, 1, 2]])
    with pytest.raises(IndexError):
        sti._view_ids_int32(qv, sv, 2, 2)  # s view 2 of 2
    a, b = sti._view_ids_int32(qv, sv, 2, 3)
    assert a.dtype == torch.int32 and b.dtype == torch.int32


def test_head_counts_run_on_built_counts_with_zero_heads():
    # 3, 5, 6, 7 heads run as 4 or 8 (4 at most in float32) with zero heads appended, which
    # leave every score unchanged (oracle scores on the padded and the plain inputs).
    from oracle import indexer as oidx
    assert [sti.kernel_heads(h, torch.bfloat16) for h in range(1, 10)] == [1, 2, 4, 4, 8, 8, 8, 8, None]
    assert [sti.kernel_heads(h, torch.float32) for h in range(1, 6)] == [1, 2, 4, 4, None]
    g = torch.Generator().manual_seed(3)
    q, k, w = torch.randn(2, 50, 3, 64, generator=g), torch.randn(2, 70, 3, 64, generator=g), torch.randn(2, 70, 3, generator=g)
    qp, kp, wp = sti.pad_heads(q, 4), sti.pad_heads(k, 4), sti.pad_heads(w, 4)
    assert qp.shape == (2, 50, 4, 64) and wp.shape == (2, 70, 4)
    assert torch.equal(qp[:, :, :3], q) and not qp[:, :, 3].any() and not wp[:, :, 3].any()
    torch.testing.assert_close(oidx.indexer_scores(qp, kp, wp, None, 0.125),
                               oidx.indexer_scores(q, k, w, None, 0.125), atol=1e-6, rtol=1e-6)
    # the backward of the real heads is the same with the zero heads present
    idx = torch.randint(0, 70, (2, 50, 8), generator=g)
    gs = torch.randn(2, 50, 8, generator=g)
    ref = oidx.indexer_topk_bwd(q, k, w, idx, gs, 0.125)
    pad = oidx.indexer_topk_bwd(qp, kp, wp, idx, gs, 0.125)
    torch.testing.assert_close(pad[0][:, :, :3], ref[0], atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(pad[1][:, :, :3], ref[1], atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(pad[2][:, :, :3], ref[2], atol=1e-6, rtol=1e-6)
