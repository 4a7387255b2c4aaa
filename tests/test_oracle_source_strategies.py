"""CPU checks of the oracle's source-downsample strategies other than "legacy"
(oracle/source_downsample.py): strategy resolution and coarse budgets by hand, the factor-4
sub-cell tables by hand and against F.avg_pool2d, the static pack by hand, exact_rerank
against the brute-force top-k when every source row is chosen, subcell_top1 and the query
downsampling on hand-built cases.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import indexer as oidx
from oracle import source_downsample as osd


def test_resolve_strategy_table():
    r = osd.resolve_strategy
    assert r("qk_sym_x2_broadcast", 2) == "qk_sym_x2_broadcast"
    assert r("qk_sym_x2_broadcast", 4) == "legacy"
    assert r("exact_rerank", 2) == "legacy" and r("subcell_top1", 3) == "legacy"
    assert r("exact_rerank", 4) == "exact_rerank" and r(" Subcell_Top1 ", 8) == "subcell_top1"
    assert r("subcell_static_pack4", 4) == "subcell_static_pack4"
    assert r("no_such_strategy", 4) == "legacy" and r(None, 4) == "legacy" and r("", 2) == "legacy"


def test_coarse_budget_for_subcell_strategies_by_hand():
    # 8 views of 20 specials + a 16 x 16 grid, factor 4: 160 specials, no edges, 128 cells, L = 288.
    lay = osd.source_layout(20 + 16 * 16, 8, 20, 4)
    assert (lay["source_len"], lay["special_count"], lay["coarse_count"]) == (288, 160, 128)
    # sub-cell expansion 4 per cell: mapped 160 + 512 = 672, avg 2.333 -> ceil(256 / 2.333 * 1.1) = 121
    # < 160 specials: 160 + ceil(96 / (16 / 4) * 1.1) = 160 + 27
    assert osd.coarse_topk_for(lay, 256, "subcell_top1") == 187
    # static pack: specials + ceil(96 / 4 * 1.1)
    assert osd.coarse_topk_for(lay, 256, "subcell_static_pack4") == 187
    assert osd.coarse_topk_for(lay, 64, "subcell_static_pack4") == 64  # 64 specials, nothing left
    # other strategies use the legacy budget; an explicit budget wins everywhere
    assert osd.coarse_topk_for(lay, 256, "exact_rerank") == osd.coarse_topk(lay, 256)
    assert osd.coarse_topk_for(lay, 256, "subcell_top1", explicit=50) == 50


def test_subcell_table_tiny_case_by_hand():
    lay = osd.source_layout(16, 1, 0, 4)
    sub = osd.subcell_table(lay)
    assert sub.tolist() == [[[0, 1, 4, 5], [2, 3, 6, 7], [8, 9, 12, 13], [10, 11, 14, 15]]]
    assert osd.subcell_table(osd.source_layout(16, 1, 0, 4, representative_points=True)) is None
    assert osd.subcell_table(osd.source_layout(64, 1, 0, 8)) is None


def test_subcell_pooling_equals_avg_pool2d():
    g = torch.Generator().manual_seed(7)
    tpv, views, psi, grid = 3 + 10 * 10, 2, 3, 10
    k = torch.randn(2, tpv * views, 2, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(2, tpv * views, 2, generator=g)).bfloat16()
    lay = osd.source_layout(tpv, views, psi, 4)
    sub = osd.subcell_table(lay)
    C = lay["coarse_count"]
    sk, sw = osd.pool_rows(k, w, sub.reshape(-1, 4))
    img = k.float().view(2, views, tpv, 128)[:, :, psi:].reshape(2 * views, grid, grid, 128).permute(0, 3, 1, 2)
    pooled = F.avg_pool2d(img[:, :, :8, :8], 2)  # [2V, 128, 4, 4]: sub-cell (2 cy + sy, 2 cx + sx)
    ref = pooled.view(2 * views, 128, 2, 2, 2, 2).permute(0, 2, 4, 3, 5, 1).reshape(2, views * 4, 4, 2, 64)
    assert torch.equal(sk.view(2, C, 4, 2, 64), ref.bfloat16())
    imgw = w.float().view(2, views, tpv, 2)[:, :, psi:].reshape(2 * views, grid, grid, 2).permute(0, 3, 1, 2)
    pw = F.avg_pool2d(imgw[:, :, :8, :8], 2).view(2 * views, 2, 2, 2, 2, 2).permute(0, 2, 4, 3, 5, 1)
    assert torch.equal(sw.view(2, C, 4, 2), pw.reshape(2, views * 4, 4, 2).bfloat16())


def test_static_pack4_table_by_hand():
    lay = osd.source_layout(1 + 16, 1, 1, 4)  # one special, one 4 x 4 cell
    sub = osd.subcell_table(lay)
    w = torch.ones(2, 1, 4, 2)
    w[0, 0, 2] = torch.tensor([1.0, 1.5])      # batch 0: sub-cell 2 has the largest mean
    w[1, 0, 1] = torch.tensor([2.0, 0.0])      # batch 1: sub-cells 0, 2, 3 mean 1, sub-cell 1 mean 1: tie -> 0
    table = osd.static_pack4_table(w.bfloat16(), lay, sub)
    assert table[0].tolist() == [[0, -1, -1, -1], [9, 10, 13, 14]]
    assert table[1].tolist() == [[0, -1, -1, -1], [1, 2, 5, 6]]


def test_rerank_with_every_row_is_the_exact_topk():
    g = torch.Generator().manual_seed(3)
    tpv, views, psi = 2 + 8 * 8, 2, 2
    n = tpv * views
    q = torch.randn(1, 5, 2, 64, generator=g).bfloat16()
    k = torch.randn(1, n, 2, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, n, 2, generator=g)).bfloat16()
    lay = osd.source_layout(tpv, views, psi, 4)
    rows = torch.arange(lay["source_len"]).repeat(1, 5, 1)
    got, cand, sc = osd.rerank(q, k, w, rows, lay, 40, 0.125)
    full = oidx.indexer_scores(q, k, w, None, 0.125)
    want = full.topk(40, dim=-1)[1]
    assert [sorted(r) for r in got[0].tolist()] == [sorted(r) for r in want[0].tolist()]
    # too few candidates for the target: None
    assert osd.rerank(q, k, w, rows[..., :2], lay, 40, 0.125) is None


def test_subcell_top1_by_hand():
    # one view: special token 0, then a 4 x 4 grid (tokens 1..16) = one cell; sub-cell 3
    # (tokens 11, 12, 15, 16) is aligned with the query, the others are orthogonal.
    lay = osd.source_layout(1 + 16, 1, 1, 4)
    sub = osd.subcell_table(lay)
    assert sub[0, 3].tolist() == [11, 12, 15, 16]
    q = torch.zeros(1, 1, 1, 64)
    q[..., 0] = 1.0
    k = torch.zeros(1, 17, 1, 64)
    k[0, :, 0, 1] = 1.0
    k[0, [11, 12, 15, 16], 0, 0] = 2.0
    w = torch.ones(1, 17, 1)
    sub_k, sub_w = osd.pool_rows(k, w, sub.reshape(-1, 4))
    rows = torch.tensor([[[1, 0]]])  # the cell first, then the special row
    out, scores, kept = osd.subcell_top1(q, sub_k.view(1, 1, 4, 1, 64), sub_w.view(1, 1, 4, 1), rows, lay, sub, 5, 1.0)
    assert out.tolist() == [[[0, 11, 12, 15, 16]]] and kept == [[(0, 3)]]
    assert scores[0, 0, 1].tolist() == [float("-inf")] * 4 and scores[0, 0, 0, 3] == 2.0
    # target 3: one sub-cell is kept and cut after two tokens; target 9: two sub-cells (3, then 0 by position)
    out3 = osd.subcell_top1(q, sub_k.view(1, 1, 4, 1, 64), sub_w.view(1, 1, 4, 1), rows, lay, sub, 3, 1.0)[0]
    assert out3.tolist() == [[[0, 11, 12]]]
    out9 = osd.subcell_top1(q, sub_k.view(1, 1, 4, 1, 64), sub_w.view(1, 1, 4, 1), rows, lay, sub, 9, 1.0)[0]
    assert out9.tolist() == [[[0, 1, 2, 5, 6, 11, 12, 15, 16]]]
    # every token: all four sub-cells, by position
    out17 = osd.subcell_top1(q, sub_k.view(1, 1, 4, 1, 64), sub_w.view(1, 1, 4, 1), rows, lay, sub, 17, 1.0)[0]
    assert out17.tolist() == [[[0] + sub[0].reshape(-1).tolist()]]
    # two cells in the grid, one chosen: 17 tokens cannot reach a target of 18
    lay2 = osd.source_layout(1 + 32, 1, 1, 4, grid_h=4, grid_w=8)
    sub2 = osd.subcell_table(lay2)
    k2 = torch.zeros(1, 33, 1, 64)
    sk2, sw2 = osd.pool_rows(k2, torch.ones(1, 33, 1), sub2.reshape(-1, 4))
    assert osd.subcell_top1(q, sk2.view(1, 2, 4, 1, 64), sw2.view(1, 2, 4, 1), rows, lay2, sub2, 18, 1.0) is None


def test_query_downsample_by_hand():
    lay = osd.source_layout(11, 2, 2, 2)  # rows as in the legacy tiny case: cells [2,3,5,6], [13,14,16,17]
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 22, 2, 8, generator=g).bfloat16()
    cq, f2l = osd.query_downsample(q, lay, 0)
    f2r = osd.fine_to_source_row(lay)
    assert cq.shape[1] == lay["source_len"]  # the whole sequence: every row is full
    cell_row = f2r[2]
    cell = [2, 3, 5, 6]
    want = (q[0, cell].float().sum(0).bfloat16().float() / 4).bfloat16()
    assert torch.equal(cq[0, f2l[2]], want)
    assert all(f2l[t] == f2l[2] for t in cell) and f2r[3] == cell_row
    single = 4  # an edge token: its own query, unchanged
    assert torch.equal(cq[0, f2l[single]], q[0, single])
    # a chunk that splits the first view's cell: tokens 0..3 -> rows of tokens 2, 3 are partial
    cq2, f2l2 = osd.query_downsample(q[:, :4], lay, 0)
    assert cq2.shape[1] == 4 and torch.equal(cq2[0, f2l2], q[0, :4])
    # the same chunk at an offset: tokens 11..21 hold the second view completely
    cq3, f2l3 = osd.query_downsample(q[:, 11:], lay, 11)
    assert cq3.shape[1] == 2 + 5 + 1 and f2l3[13 - 11] == f2l3[17 - 11]


def test_qk_sym_broadcasts_one_selection_per_cell():
    g = torch.Generator().manual_seed(9)
    tpv, views, psi = 1 + 6 * 6, 2, 1
    n = tpv * views
    q = torch.randn(1, n, 2, 64, generator=g).bfloat16()
    k = torch.randn(1, n, 2, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, n, 2, generator=g)).bfloat16()
    lay = osd.source_layout(tpv, views, psi, 2)
    out = osd.select_strategy(q, k, w, lay, 20, 0.125, "qk_sym_x2_broadcast")
    f2r = osd.fine_to_source_row(lay)
    off = lay["special_count"] + lay["edge_count"]
    for r in range(off, lay["source_len"]):
        toks = [t for t in lay["source_to_fine"][r] if t >= 0]
        assert all(torch.equal(out[0, t], out[0, toks[0]]) for t in toks)
    assert out.shape == (1, n, 20) and (f2r >= 0).all()


def test_strategy_fallbacks():
    g = torch.Generator().manual_seed(4)
    tpv, views, psi = 1 + 8 * 8, 1, 1
    q = torch.randn(1, 3, 2, 64, generator=g).bfloat16()
    k = torch.randn(1, tpv * views, 2, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, tpv * views, 2, generator=g)).bfloat16()
    lay = osd.source_layout(tpv, views, psi, 4, representative_points=True)
    full = oidx.indexer_scores(q, k, w, None, 0.125).topk(16, dim=-1)[1]
    # no sub-cell keys with representative points: both sub-cell strategies end on the full indexer
    for s in ("subcell_static_pack4", "subcell_top1"):
        got = osd.select_strategy(q, k, w, lay, 16, 0.125, s)
        assert [sorted(r) for r in got[0].tolist()] == [sorted(r) for r in full[0].tolist()]
    # exact_rerank with representative points reranks the 4 points of each chosen cell
    got = osd.select_strategy(q, k, w, lay, 16, 0.125, "exact_rerank")
    assert got.shape == (1, 3, 16)
