"""GPU parity of the source-downsample strategies other than "legacy" against the oracle
restatement (oracle/source_downsample.py): the 2 x 2 sub-cell keys, the query means and the
static pack tables bit-exact; exact_rerank and subcell_top1 on given chosen rows against the
oracle (tie-aware where scores decide, exact where they do not); the selector's steps wired
as the reference's dispatch runs them (retries included); qk_sym_x2_broadcast's query cells
and broadcast bit-exact.
"""
import math

import numpy as np
import pytest
import torch

from geoweave_amd import source_downsample as sd
from geoweave_amd.custom_indexer import sparse_topk_indexer_inference_func
from oracle import indexer as oidx
from oracle import source_downsample as osd
from oracle.topk_check import check_topk_rows

pytestmark = pytest.mark.gpu

SCALE = 0.125


def _inputs(tpv, views, seed, dtype=torch.bfloat16, B=1, T=None):
    g = torch.Generator().manual_seed(seed)
    n = tpv * views
    q = torch.randn(B, n if T is None else T, 4, 64, generator=g).to(dtype)
    k = torch.randn(B, n, 4, 64, generator=g).to(dtype)
    w = (1 + 0.3 * torch.randn(B, n, 4, generator=g)).to(dtype)
    return q, k, w


def _coarse(qd, prep, n):
    return sparse_topk_indexer_inference_func(qd, prep.source_k, prep.source_w, qd.new_empty(0), n, SCALE, 256, 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_subcell_keys_and_static_table_bit_exact(gpu_device, dtype):
    tpv, views, psi = 5 + 37 * 37, 2, 5
    q, k, w = _inputs(tpv, views, 5, dtype, B=2)
    lay = osd.source_layout(tpv, views, psi, 4)
    sub = osd.subcell_table(lay)
    for strategy in ("subcell_top1", "subcell_static_pack4"):
        cfg = sd.SourceDownsample(tpv, views, psi, factor=4, strategy=strategy)
        prep = sd.prepare(k.cuda(), w.cuda(), cfg)
        assert np.array_equal(prep.layout.subcell_to_fine, sub.reshape(-1, 4))
        rk, rw = osd.pool_rows(k, w, sub.reshape(-1, 4))
        torch.cuda.synchronize()
        if strategy == "subcell_top1":
            assert torch.equal(prep.sub_k.cpu(), rk) and torch.equal(prep.sub_w.cpu(), rw)
        else:
            want = osd.static_pack4_table(rw.view(2, -1, 4, 4), lay, sub)
            assert np.array_equal(prep.static_table.cpu().numpy(), want)


@pytest.mark.parametrize("q_offset,n", [(0, 2 * (5 + 37 * 37)), (700, 1500), (3, 40)])
def test_query_downsample_bit_exact(gpu_device, q_offset, n):
    tpv, views, psi = 5 + 37 * 37, 2, 5
    q, _, _ = _inputs(tpv, views, 8, B=2)
    qc = q[:, q_offset:q_offset + n]
    cfg = sd.SourceDownsample(tpv, views, psi, factor=2, strategy="qk_sym_x2_broadcast")
    cq, f2l = sd.query_downsample(qc.cuda(), cfg, q_offset)
    lay = osd.source_layout(tpv, views, psi, 2)
    rq, rf2l = osd.query_downsample(qc, lay, q_offset)
    torch.cuda.synchronize()
    assert np.array_equal(f2l.cpu().numpy(), rf2l)
    assert torch.equal(cq.cpu(), rq)


@pytest.mark.parametrize("rep,dtype,target", [(False, torch.bfloat16, 700), (True, torch.bfloat16, 300),
                                              (False, torch.float16, 512)])
def test_rerank_given_rows(gpu_device, rep, dtype, target):
    tpv, views, psi = 5 + 37 * 37, 2, 5
    T = 48
    q, k, w = _inputs(tpv, views, 13, dtype, B=2, T=T)
    cfg = sd.SourceDownsample(tpv, views, psi, factor=4, representative_points=rep, strategy="exact_rerank")
    layout = sd.build_layout(cfg)
    table = torch.from_numpy(layout.source_to_fine).cuda()
    lay = osd.source_layout(tpv, views, psi, 4, representative_points=rep)
    g = torch.Generator().manual_seed(2)
    Kc = 150 if not rep else 200  # at least 1125 (476) candidates per query
    cidx = torch.stack([torch.randperm(layout.source_len, generator=g)[:Kc] for _ in range(2 * T)]).view(2, T, Kc)
    out, ok = sd.rerank(q.cuda(), k.cuda(), w.cuda(), cidx.cuda(), layout, table, target, SCALE)
    assert ok
    got = out.cpu().long()
    res = osd.rerank(q, k, w, cidx, lay, target, SCALE)
    assert res is not None
    _, cand, sc = res
    n = tpv * views
    for b in range(2):
        # scores over every fine token, -inf for the tokens that are not candidates
        full = torch.full((T, n), float("-inf"))
        for t in range(T):
            ok_t = cand[b, t] >= 0
            full[t, cand[b, t][ok_t]] = sc[b, t][ok_t]
        rep_ = check_topk_rows(full, got[b], target)
        assert rep_.ok, rep_.first_bad
    # a target above every query's candidates: the fail flag
    _, ok_small = sd.rerank(q.cuda(), k.cuda(), w.cuda(), cidx[..., :4].cuda(), layout, table,
                            min(4 * layout.max_block_tokens, target), SCALE)
    few = osd.rerank(q, k, w, cidx[..., :4], lay, min(4 * layout.max_block_tokens, target), SCALE)
    assert ok_small == (few is not None)


@pytest.mark.parametrize("dtype,target", [(torch.bfloat16, 600), (torch.float16, 257), (torch.bfloat16, 64)])
def test_subcell_top1_given_rows(gpu_device, dtype, target):
    tpv, views, psi = 20 + 36 * 36, 2, 20
    T = 40
    q, k, w = _inputs(tpv, views, 17, dtype, B=2, T=T)
    cfg = sd.SourceDownsample(tpv, views, psi, factor=4, strategy="subcell_top1")
    prep = sd.prepare(k.cuda(), w.cuda(), cfg)
    layout = prep.layout
    lay = osd.source_layout(tpv, views, psi, 4)
    sub = osd.subcell_table(lay)
    g = torch.Generator().manual_seed(4)
    Kc = 120  # of 40 special rows and 162 cells
    # chosen rows: always some special rows (< 40) among them
    cidx = torch.stack([torch.cat([torch.randperm(40, generator=g)[:12],
                                   40 + torch.randperm(layout.source_len - 40, generator=g)[:Kc - 12]])
                        for _ in range(2 * T)]).view(2, T, Kc)
    csc = torch.randn(2, T, Kc, generator=g).to(dtype)
    out, ok = sd.subcell_top1(q.cuda(), prep.sub_k, prep.sub_w, cidx.cuda(), csc.cuda(), layout, prep.table,
                              prep.sub_table, target, SCALE)
    assert ok
    rows = osd.order_by_score(cidx, csc)
    rk, rw = osd.pool_rows(k, w, sub.reshape(-1, 4))
    C = lay["coarse_count"]
    res = osd.subcell_top1(q, rk.view(2, C, 4, 4, 64), rw.view(2, C, 4, 4), rows, lay, sub, target, SCALE)
    assert res is not None
    want, scores, _ = res
    got = out.cpu().long()
    mismatched = 0
    for b in range(2):
        for t in range(T):
            if torch.equal(got[b, t], want[b, t]):
                continue
            # only a near-tie at the kept/dropped boundary may pick another sub-cell
            s = scores[b, t].reshape(-1)
            s = s[torch.isfinite(s)].sort(descending=True).values
            singles = sum(1 for r in rows[b, t].tolist() if r < lay["special_count"] + lay["edge_count"])
            keep = min(math.ceil(max(target - singles, 0) / 4), s.numel())
            assert 0 < keep < s.numel(), (b, t)
            gap = float(s[keep - 1] - s[keep])
            assert gap <= 1e-5 * max(abs(float(s[keep - 1])), 1.0), (b, t, gap)
            mismatched += 1
    assert mismatched <= 2
    # too few tokens for the target: the fail flag, as the oracle
    small = cidx[..., :3]
    _, ok2 = sd.subcell_top1(q.cuda(), prep.sub_k, prep.sub_w, small.cuda(), csc[..., :3].cuda(), layout, prep.table,
                             prep.sub_table, 40, SCALE)
    assert not ok2 and osd.subcell_top1(q, rk.view(2, C, 4, 4, 64), rw.view(2, C, 4, 4),
                                        osd.order_by_score(small, csc[..., :3]), lay, sub, 40, SCALE) is None


@pytest.mark.parametrize("strategy", ["exact_rerank", "subcell_top1", "subcell_static_pack4"])
def test_selector_runs_the_reference_dispatch(gpu_device, strategy):
    # The selector's output equals its steps run by hand: the coarse top-k at the strategy's
    # budget, grown by recall_growth while a query is short of candidates (a small explicit
    # budget forces at least one retry), then the strategy's kernel.
    tpv, views, psi, topk = 5 + 37 * 37, 2, 5, 512
    q, k, w = _inputs(tpv, views, 23)
    qd, kd, wd = q.cuda(), k.cuda(), w.cuda()
    explicit = 20 if strategy != "subcell_static_pack4" else 0
    cfg = sd.SourceDownsample(tpv, views, psi, factor=4, strategy=strategy, coarse_topk=explicit, query_chunk=1000)
    fine = sd.select_topk(qd, kd, wd, topk, SCALE, cfg)
    prep = sd.prepare(kd, wd, cfg)
    layout = prep.layout
    lay = osd.source_layout(tpv, views, psi, 4)
    kc = sd.coarse_budget(layout, topk, cfg)
    assert kc == osd.coarse_topk_for(lay, topk, strategy, explicit=explicit)
    T = q.shape[1]
    parts = []
    retries = 0
    for s0 in range(0, T, 1000):
        qc = qd[:, s0:s0 + 1000].contiguous()
        if strategy == "subcell_static_pack4":
            cidx, csc = _coarse(qc, prep, kc)
            parts.append(sd.expand(cidx, layout, prep.static_table, topk, 64, csc, round_robin=True))
            continue
        attempt, out = kc, None
        for _ in range(cfg.recall_max_steps):
            cidx, csc = _coarse(qc, prep, attempt)
            if strategy == "exact_rerank":
                out, ok = sd.rerank(qc, kd, wd, cidx, layout, prep.table, topk, SCALE)
            else:
                out, ok = sd.subcell_top1(qc, prep.sub_k, prep.sub_w, cidx, csc, layout, prep.table, prep.sub_table,
                                          topk, SCALE)
            if ok:
                break
            out = None
            retries += 1
            if attempt >= layout.source_len:
                break
            attempt = min(max(math.ceil(attempt * 1.5), attempt + 1), layout.source_len)
        if out is None:  # every attempt short of candidates: the full indexer
            out, _ = sparse_topk_indexer_inference_func(qc, kd, wd, qc.new_empty(0), topk, SCALE, 256, 0)
        parts.append(out)
    torch.cuda.synchronize()
    assert torch.equal(fine, torch.cat(parts, 1))
    if strategy != "subcell_static_pack4":
        assert retries >= 1
    if strategy == "subcell_static_pack4":
        # the expansion of the GPU's coarse rows through the oracle's per-batch table
        sub = osd.subcell_table(lay)
        _, rw = osd.pool_rows(k, w, sub.reshape(-1, 4))
        table = osd.static_pack4_table(rw.view(1, -1, 4, 4), lay, sub)
        cidx, csc = _coarse(qd, prep, kc)
        want = osd.expand(osd.order_by_score(cidx.cpu(), csc.cpu()), dict(lay, source_to_fine=table[0]), topk,
                          tpv * views)
        assert torch.equal(fine.cpu().long(), want)
    # valid tokens per query, distinct where no padding repeats them (the static pack's
    # expansion pads a query short of tokens with repeats, as the reference's does)
    assert int(fine.min()) >= 0 and int(fine.max()) < tpv * views
    if strategy != "subcell_static_pack4":
        srt = fine.sort(-1).values
        assert not bool((srt[..., 1:] == srt[..., :-1]).any())


def test_subcell_strategies_fall_back_without_subcell_keys(gpu_device):
    # representative points: no sub-cell keys, so the full indexer answers (as the reference)
    tpv, views, psi, topk = 5 + 37 * 37, 2, 5, 256
    q, k, w = _inputs(tpv, views, 29, T=64)
    qd, kd, wd = q.cuda(), k.cuda(), w.cuda()
    full, _ = sparse_topk_indexer_inference_func(qd, kd, wd, qd.new_empty(0), topk, SCALE, 256, 0)
    for strategy in ("subcell_top1", "subcell_static_pack4"):
        cfg = sd.SourceDownsample(tpv, views, psi, factor=4, representative_points=True, strategy=strategy)
        assert torch.equal(sd.select_topk(qd, kd, wd, topk, SCALE, cfg), full)
    # factor 8 without representative points: the reference's sub-cell reshape fails; here a ValueError
    n8 = 2 * (5 + 40 * 40)
    with pytest.raises(ValueError):
        sd.prepare(torch.zeros(1, n8, 4, 64, dtype=torch.bfloat16, device="cuda"),
                   torch.zeros(1, n8, 4, dtype=torch.bfloat16, device="cuda"),
                   sd.SourceDownsample(5 + 40 * 40, 2, 5, factor=8, strategy="subcell_top1"))


@pytest.mark.parametrize("chunk", [0, 900])
def test_qk_sym_matches_oracle(gpu_device, chunk):
    tpv, views, psi, topk = 5 + 37 * 37, 2, 5, 512
    q, k, w = _inputs(tpv, views, 31)
    qd, kd, wd = q.cuda(), k.cuda(), w.cuda()
    cfg = sd.SourceDownsample(tpv, views, psi, factor=2, strategy="qk_sym_x2_broadcast", query_chunk=chunk)
    fine = sd.select_topk(qd, kd, wd, topk, SCALE, cfg)
    prep = sd.prepare(kd, wd, cfg)
    lay = osd.source_layout(tpv, views, psi, 2)
    kc = sd.coarse_budget(prep.layout, topk, cfg)
    T = q.shape[1]
    step = T if chunk == 0 else chunk
    rk, rw = osd.pool_sources(k, w, lay)
    for s0 in range(0, T, step):
        cq, f2l = sd.query_downsample(qd[:, s0:s0 + step].contiguous(), cfg, s0)
        cidx, csc = _coarse(cq, prep, kc)
        # coarse sets tie-aware against the oracle scores of the (bit-exact) coarse queries
        rq, rf2l = osd.query_downsample(q[:, s0:s0 + step], lay, s0)
        assert torch.equal(cq.cpu(), rq)
        rows = torch.arange(0, cq.shape[1], 7)
        sc = oidx.indexer_scores(rq[:, rows], rk, rw, None, SCALE)
        rep = check_topk_rows(sc[0], cidx[0, rows].cpu(), kc)
        assert rep.ok, rep.first_bad
        # the broadcast expansion: bit-exact
        want = osd.expand(osd.order_by_score(cidx.cpu(), csc.cpu()), lay, topk, tpv * views)[:, torch.from_numpy(rf2l)]
        assert torch.equal(fine[:, s0:s0 + step].cpu().long(), want)


@pytest.mark.parametrize("factor,strategy", [(4, "exact_rerank"), (4, "subcell_top1"), (4, "subcell_static_pack4"),
                                             (2, "qk_sym_x2_broadcast")])
def test_layer_runs_each_strategy(gpu_device, factor, strategy):
    from geoweave_amd import dsa_layer, workloads

    torch.manual_seed(0)
    views, topk = 2, 256
    m = workloads.init_layer_(dsa_layer.SparseGlobalAttention(topk=topk)).cuda()
    x, pos = workloads.layer_module_inputs(views)
    x, pos = x.cuda(), pos.cuda()
    N = x.shape[1]
    cfg = sd.SourceDownsample(tokens_per_view=N // views, num_views=views, patch_start_idx=5, factor=factor,
                              strategy=strategy)
    with torch.no_grad():
        out, idx = m(x, pos, return_topk=True, source_downsample=cfg)
        again = m(x, pos, topk_indices=idx)
    torch.cuda.synchronize()
    assert idx.shape == (1, N, topk) and int(idx.min()) >= 0 and int(idx.max()) < N
    assert bool(torch.isfinite(out.float()).all()) and torch.equal(out, again)


def test_stream_with_qk_sym_takes_the_selector_chunk(gpu_device):
    # dsa_attention.py:870-881,1127-1136: with qk_sym_x2_broadcast the stream's outer chunk is
    # min(N, source_downsample_query_chunk), not the layer's query chunk; a layer chunk of 700
    # (a source cell straddles token 700) must give the rows of 1024-token selector chunks.
    from geoweave_amd import dsa_layer, workloads
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import sparse_index_flash_attn_inference_func

    tpv, views, psi, topk, qc = 5 + 37 * 37, 2, 5, 512, 1024
    q, k, w = _inputs(tpv, views, 33)
    N = q.shape[1]
    aq, ak, av = (x.cuda() for x in workloads.attention_inputs(1, 1, torch.bfloat16, tokens=N, seed=34))
    qd, kd, wd = q.cuda(), k.cuda(), w.cuda()
    cfg = sd.SourceDownsample(tpv, views, psi, factor=2, strategy="qk_sym_x2_broadcast", query_chunk=qc)
    o = dsa_layer.sparse_attention_streaming(aq, ak, av, qd, kd, wd, topk, 700, SCALE, 0.125, cfg)

    def chunked(step):
        return torch.cat([sd.select_topk(qd[:, s0:s0 + step].contiguous(), kd, wd, topk, SCALE, cfg, q_offset=s0)
                          for s0 in range(0, N, step)], dim=1)

    idx = chunked(qc)
    o_ref, _ = sparse_index_flash_attn_inference_func(aq, ak, av, idx, softmax_scale=0.125)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    # the layer's chunking would select other rows (cells cut at 700)
    assert not torch.equal(chunked(700), idx)
