"""GPU parity of the fused indexer score + exact top-k against the fp32 CPU oracle.

Bar: index sets bit-exact except where oracle fp32 scores tie within 1e-6 relative
(oracle/topk_check.py); returned scores within 2e-2 of the oracle's selected scores.
"""
import json
from pathlib import Path

import pytest
import torch

from geoweave_amd import workloads
from geoweave_amd.custom_indexer import sparse_topk_indexer as sti
from oracle import indexer as oidx
from oracle.topk_check import check_topk_rows

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _gpu_topk(q, k, w, topk, scale=0.125, mask=None, flags=0, dev="cuda"):
    m = None if mask is None else mask.to(dev)
    idx, sc = sti.indexer_topk_forward(q.to(dev), k.to(dev), w.to(dev), m, topk, scale, flags)
    torch.cuda.synchronize()
    return idx.cpu(), sc.cpu()


def _check(q, k, w, idx, sc, topk, scale=0.125, mask=None, rows=None):
    """Tie-aware set check over every (or the given) row, plus score values."""
    B = q.shape[0]
    for b in range(B):
        qb = q[b:b + 1] if rows is None else q[b:b + 1, rows]
        mb = None if mask is None else (mask[b:b + 1] if rows is None else mask[b:b + 1, rows])
        ref = oidx.indexer_scores(qb, k[b:b + 1], w[b:b + 1], mb, scale)[0]
        got = idx[b] if rows is None else idx[b, rows]
        rep = check_topk_rows(ref, got, topk)
        assert rep.ok, f"batch {b}: {rep}"
        gs = sc[b] if rows is None else sc[b, rows]
        torch.testing.assert_close(gs.float(), ref.gather(1, got.long()), atol=2e-2, rtol=2e-2)
    return rep


@pytest.mark.parametrize("case", json.loads((GOLDEN / "indexer_kat.json").read_text()), ids=lambda c: c["name"])
def test_golden_kat_zero_padded(gpu_device, case):
    # The reference test's tiny q/k (Di = 2 or 3) zero-padded to Di = 64: same scores.
    q = torch.tensor(case["q"]).unsqueeze(0)
    k = torch.tensor(case["k"]).unsqueeze(0)
    w = torch.tensor(case["w"]).unsqueeze(0)
    pad = 64 - q.shape[-1]
    q = torch.nn.functional.pad(q, (0, pad)).bfloat16()
    k = torch.nn.functional.pad(k, (0, pad)).bfloat16()
    w = w.bfloat16()
    mask = None if case["mask"] is None else torch.tensor(case["mask"]).unsqueeze(0).bfloat16()
    idx, sc = _gpu_topk(q, k, w, case["topk"], case["scale"], mask)
    ref = torch.tensor(case["scores"], dtype=torch.float32)
    rep = check_topk_rows(ref, idx[0], case["topk"])
    assert rep.ok, rep
    if case["name"].startswith("reference"):
        assert [sorted(r) for r in idx[0].tolist()] == case["expected_sets"]


@pytest.mark.parametrize("views,topk", [(1, 1024), (1, 256), (4, 1024)])
def test_layer_inputs_bf16(gpu_device, views, topk):
    q, k, w = workloads.indexer_inputs(views, 1, torch.bfloat16)
    idx, sc = _gpu_topk(q, k, w, topk)
    assert idx.shape == (1, q.shape[1], topk) and idx.dtype == torch.int32 and sc.dtype == torch.bfloat16
    rep = _check(q, k, w, idx, sc, topk)
    print(f"views={views} topk={topk}: exact rows {rep.rows_exact}/{rep.rows}, tie-swapped {rep.rows_tie_swapped}")


def test_layer_inputs_fp16_batch2(gpu_device):
    q, k, w = workloads.indexer_inputs(2, 2, torch.float16)
    idx, sc = _gpu_topk(q, k, w, 512)
    _check(q, k, w, idx, sc, 512)


def test_sampled_path_batch3_ragged_rows(gpu_device):
    # B = 3 with T = 4500 (not a multiple of the 32-row candidate groups) and S > 4096 (the
    # sampled threshold): every row of every batch element is checked.
    q, k, w = workloads.indexer_inputs(4, 3, torch.bfloat16, tokens=4500)
    idx, sc = _gpu_topk(q, k, w, 1024)
    _check(q, k, w, idx, sc, 1024)


@pytest.mark.parametrize("heads", [1, 2, 8])
def test_other_head_counts(gpu_device, heads):
    g = torch.Generator().manual_seed(heads)
    n = 5000
    q = torch.randn(1, n, heads, 64, generator=g).bfloat16()
    k = torch.randn(1, n, heads, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, n, heads, generator=g)).bfloat16()
    idx, sc = _gpu_topk(q, k, w, 300, scale=0.125)
    _check(q, k, w, idx, sc, 300)


def test_additive_mask(gpu_device):
    q, k, w = workloads.indexer_inputs(1, 1, torch.bfloat16, tokens=2000)
    g = torch.Generator().manual_seed(3)
    mask = torch.randn(1, 2000, 2000, generator=g)
    mask[torch.rand(1, 2000, 2000, generator=g) < 0.2] = float("-inf")
    mask = mask.bfloat16()
    idx, sc = _gpu_topk(q, k, w, 400, mask=mask)
    _check(q, k, w, idx, sc, 400, mask=mask.float())


@pytest.mark.parametrize("flags,tokens", [(sti.FLAG_TAU_PLUS_INF, None), (sti.FLAG_TAU_MINUS_INF, None),
                                          (sti.FLAG_TAU_MINUS_INF, 12000), (sti.FLAG_FORCE_WIDE, None),
                                          (sti.FLAG_FORCE_WIDE, 2000)])
def test_forced_fallback_paths_are_exact(gpu_device, flags, tokens):
    # PLUS_INF: no candidate passes, every query takes the brute-force path.
    # MINUS_INF at N=5496: every key is a candidate and the lists hold them all.
    # MINUS_INF at N=12000: every key passes and the query's candidate lists
    # (8192 slots per query) overflow, so every query takes the brute-force path.
    # FORCE_WIDE: every query is selected by the LDS path (with sampling at N=5496,
    # without at N=2000) instead of the register path.
    q, k, w = workloads.indexer_inputs(4, 1, torch.bfloat16, tokens=tokens)
    if tokens is not None:
        q = q[:, :1024].contiguous()
    idx, sc = _gpu_topk(q, k, w, 1024, flags=flags)
    _check(q, k, w, idx, sc, 1024)


@pytest.mark.parametrize("S,topk,T", [(40000, 2048, 300), (40000, 4096, 200), (12000, 3000, 700),
                                      (12000, 5000, 400), (9500, 9000, 600)])
def test_topk_above_the_register_and_candidate_slots(gpu_device, S, topk, T):
    # No step bounds the top-k: at S = 40,000, k = 2,048 and 4,096 expect ≈ 3,000 and 5,400
    # candidates, which the 64- and 96-slot register selects hold; past those slots rows take
    # the LDS selection, and where the lists would overflow every row is scored over every
    # key on the matrix cores. Every row against the oracle, then the backward (the CSR path above k = 2,048)
    # against the oracle on the GPU's indices.
    from geoweave_amd.custom_indexer._backward import indexer_topk_backward
    g = torch.Generator().manual_seed(topk)
    q = torch.randn(1, T, 4, 64, generator=g).bfloat16()
    k = torch.randn(1, S, 4, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, S, 4, generator=g)).bfloat16()
    print(f"[indexer] topk={topk} S={S} T={T}", flush=True)
    idx, sc = _gpu_topk(q, k, w, topk)
    assert idx.shape == (1, T, topk)
    _check(q, k, w, idx, sc, topk)
    gs = torch.randn(1, T, topk, generator=g).bfloat16()
    dq, dk, dw = indexer_topk_backward(q.cuda(), k.cuda(), w.cuda(), idx.cuda(), gs.cuda(), 0.125)
    torch.cuda.synchronize()
    rq, rk, rw = oidx.indexer_topk_bwd(q, k, w, idx.long(), gs.float(), 0.125)
    for got, ref in ((dq, rq), (dk, rk), (dw, rw)):
        bad = ~torch.isclose(got.float().cpu(), ref, atol=2e-2, rtol=2e-2)
        assert bad.float().mean() <= 1e-3, f"{int(bad.sum())} of {bad.numel()} outside tolerance"


def test_topk_above_the_candidate_slots_with_a_mask(gpu_device):
    # The brute-force path (every row at k = 9,000 > 8,192 candidate slots) adds the additive
    # mask too; -inf entries included.
    g = torch.Generator().manual_seed(9)
    T, S, topk = 300, 9500, 9000
    q = torch.randn(1, T, 4, 64, generator=g).bfloat16()
    k = torch.randn(1, S, 4, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, S, 4, generator=g)).bfloat16()
    mask = torch.randn(1, T, S, generator=g)
    mask[torch.rand(1, T, S, generator=g) < 0.02] = float("-inf")
    mask = mask.bfloat16()
    idx, sc = _gpu_topk(q, k, w, topk, mask=mask)
    _check(q, k, w, idx, sc, topk, mask=mask.float())


def test_topk_full_rows_path_in_rounds_with_view_bias(gpu_device):
    # k = 8,000 of 9,000 keys: every row is scored over every key and selected exactly, in
    # rounds of 512 rows per batch element (1,100 rows: three rounds, the last partial), with
    # the soft view bias on every score.
    g = torch.Generator().manual_seed(12)
    B, T, S, topk, Vq, Vs = 2, 1100, 9000, 8000, 3, 5
    q = torch.randn(B, T, 4, 64, generator=g).bfloat16()
    k = torch.randn(B, S, 4, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(B, S, 4, generator=g)).bfloat16()
    qv = torch.randint(0, Vq, (B, T), generator=g, dtype=torch.int32)
    sv = torch.randint(0, Vs, (B, S), generator=g, dtype=torch.int32)
    table = torch.randn(B, Vq, Vs, generator=g).bfloat16()
    idx, sc = sti.indexer_topk_forward(q.cuda(), k.cuda(), w.cuda(), None, topk, 0.125,
                                       view_bias=(qv.cuda(), sv.cuda(), table.cuda()))
    torch.cuda.synchronize()
    idx, sc = idx.cpu(), sc.cpu()
    for b in range(B):
        ref = oidx.indexer_scores(q[b:b + 1], k[b:b + 1], w[b:b + 1], None, 0.125,
                                  view_bias=(qv[b:b + 1], sv[b:b + 1], table[b:b + 1].float()))[0]
        rep = check_topk_rows(ref, idx[b], topk)
        assert rep.ok, f"batch {b}: {rep}"
        torch.testing.assert_close(sc[b].float(), ref.gather(1, idx[b].long()), atol=2e-2, rtol=2e-2)


def test_topk_at_least_source_length(gpu_device):
    q, k, w = workloads.indexer_inputs(1, 1, torch.bfloat16, tokens=300)
    idx, sc = _gpu_topk(q, k, w, 1024)
    assert idx.shape == (1, 300, 300)
    assert torch.equal(idx[0].long().sort(-1).values, torch.arange(300).expand(300, 300))


def test_deterministic_and_stream_aware(gpu_device):
    q, k, w = workloads.indexer_inputs(4, 1, torch.bfloat16)
    a = _gpu_topk(q, k, w, 1024)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        b = _gpu_topk(q, k, w, 1024)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_dropin_entry_points(gpu_device):
    q, k, w = workloads.indexer_inputs(1, 1, torch.bfloat16)
    qd, kd, wd = q.cuda(), k.cuda(), w.cuda()
    i1, s1 = sti.sparse_topk_indexer_func(qd, kd, wd, qd.new_empty(0), 1024, 0.125, 256, 0)
    i2, s2 = sti.sparse_topk_indexer_inference_func(qd, kd, wd, qd.new_empty(0), 1024, 0.125, 256, 0,
                                                     outer_query_chunk=0, return_scores=True)
    assert torch.equal(i1, i2) and torch.equal(s1, s2)
    # a view-bias dict without its three keys is no view bias (reference :635-636)
    i3, s3 = sti.sparse_topk_indexer_func(qd, kd, wd, None, 1024, 0.125, 256, 0, view_bias_data={})
    assert torch.equal(i1, i3) and torch.equal(s1, s3)


def _pad64(x):
    return torch.nn.functional.pad(x, (0, 64 - x.shape[-1]))


@pytest.mark.parametrize("case", json.loads((GOLDEN / "indexer_view_bias_kat.json").read_text()),
                         ids=lambda c: c["name"])
def test_view_bias_golden_kat(gpu_device, case):
    # The reference's view-bias cases (tests/indexer_projected_tests.py:64-243), q/k
    # zero-padded to Di = 64, through the drop-in with view_bias_data: index sets against the
    # fp64 fixture scores (tie-aware), and d sum(topk_scores) / d view_bias counted by hand.
    dev = "cuda"
    q = _pad64(torch.tensor(case["q"]).unsqueeze(0)).bfloat16().to(dev).requires_grad_()
    k = _pad64(torch.tensor(case["k"]).unsqueeze(0)).bfloat16().to(dev).requires_grad_()
    w = torch.tensor(case["w"]).unsqueeze(0).bfloat16().to(dev).requires_grad_()
    mask = None if case["mask"] is None else torch.tensor(case["mask"]).unsqueeze(0).bfloat16().to(dev)
    table = torch.tensor(case["view_bias"], device=dev, requires_grad=True)  # fp32 [1, Vq, Vs]
    vbd = dict(q_view_ids=torch.tensor(case["q_view_ids"], device=dev),
               s_view_ids=torch.tensor(case["s_view_ids"], device=dev), view_bias=table)
    idx, sc = sti.sparse_topk_indexer_func(q, k, w, mask, case["topk"], case["scale"], 256, 0, view_bias_data=vbd)
    ref = torch.tensor(case["scores"], dtype=torch.float32)
    rep = check_topk_rows(ref, idx[0].cpu(), case["topk"])
    assert rep.ok, rep
    torch.testing.assert_close(sc[0].float().cpu(), ref.gather(1, idx[0].long().cpu()), atol=2e-2, rtol=2e-2)
    if "table_grad_of_sum" in case:
        sc.float().sum().backward()
        assert table.grad.dtype == torch.float32
        torch.testing.assert_close(table.grad.cpu(), torch.tensor(case["table_grad_of_sum"]), atol=0, rtol=0)


def _views(n, per_view):
    return (torch.arange(n) // per_view).to(torch.int64)


@pytest.mark.parametrize("with_mask", [False, True])
def test_view_bias_layer_inputs(gpu_device, with_mask):
    # S = 4 views of 1374 tokens (B = 1) or 2 x 1000-token batch elements with a mask; a
    # table of N(0, 2) entries moves many selections across views.
    if with_mask:
        q, k, w = workloads.indexer_inputs(1, 2, torch.bfloat16, tokens=2000)
        per = 500
    else:
        q, k, w = workloads.indexer_inputs(4, 1, torch.bfloat16)
        per = 1374
    B, N = q.shape[:2]
    g = torch.Generator().manual_seed(21)
    nv = (N + per - 1) // per
    table = (2 * torch.randn(B, nv, nv, generator=g)).bfloat16()
    qv = _views(N, per).expand(B, N).contiguous()
    sv = _views(N, per).flip(0).expand(B, N).contiguous()  # key views in another order
    mask = None
    if with_mask:
        mask = torch.randn(B, N, N, generator=g)
        mask[torch.rand(B, N, N, generator=g) < 0.1] = float("-inf")
        mask = mask.bfloat16()
    topk = 512
    dev = "cuda"
    qv32, sv32 = qv.to(torch.int32).to(dev), sv.to(torch.int32).to(dev)
    idx, sc = sti.indexer_topk_forward(q.to(dev), k.to(dev), w.to(dev), None if mask is None else mask.to(dev),
                                       topk, 0.125, view_bias=(qv32, sv32, table.to(dev)))
    idx, sc = idx.cpu(), sc.cpu()
    for b in range(B):
        ref = oidx.indexer_scores(q[b:b + 1], k[b:b + 1], w[b:b + 1], None if mask is None else mask[b:b + 1].float(),
                                  0.125, view_bias=(qv[b:b + 1], sv[b:b + 1], table[b:b + 1]))[0]
        rep = check_topk_rows(ref, idx[b], topk)
        assert rep.ok, f"batch {b}: {rep}"
        torch.testing.assert_close(sc[b].float(), ref.gather(1, idx[b].long()), atol=2e-2, rtol=2e-2)
    # the bias changed the selection (a test of the term, not of the plain top-k again)
    plain, _ = _gpu_topk(q, k, w, topk, mask=mask)
    assert not torch.equal(plain.sort(-1).values, idx.sort(-1).values)


@pytest.mark.parametrize("flags", [sti.FLAG_TAU_PLUS_INF, sti.FLAG_FORCE_WIDE])
def test_view_bias_forced_fallback_paths(gpu_device, flags):
    # the brute-force path (every query) and the LDS select path include the bias too
    q, k, w = workloads.indexer_inputs(4, 1, torch.bfloat16)
    q = q[:, :768].contiguous()
    N = k.shape[1]
    g = torch.Generator().manual_seed(22)
    table = (3 * torch.randn(1, 2, 4, generator=g)).bfloat16()
    qv = (torch.arange(768) % 2).view(1, -1)
    sv = _views(N, 1374).view(1, -1)
    dev = "cuda"
    idx, sc = sti.indexer_topk_forward(q.to(dev), k.to(dev), w.to(dev), None, 1024, 0.125, flags,
                                       view_bias=(qv.to(torch.int32).to(dev), sv.to(torch.int32).to(dev),
                                                  table.to(dev)))
    ref = oidx.indexer_scores(q, k, w, None, 0.125, view_bias=(qv, sv, table))[0]
    rep = check_topk_rows(ref, idx[0].cpu(), 1024)
    assert rep.ok, rep
    torch.testing.assert_close(sc[0].float().cpu(), ref.gather(1, idx[0].long().cpu()), atol=2e-2, rtol=2e-2)


def test_view_bias_gradients(gpu_device):
    # A learnable [Vq, Vs] table broadcast over B = 2 (the soft view-bias training path):
    # its gradient against the oracle's scatter (fp32 sums over the GPU's own selection,
    # summed over the batch as the broadcast does); dq/dk/dw equal the plain backward's on
    # the same selection (the bias does not enter them).
    q, k, w = workloads.indexer_inputs(1, 2, torch.bfloat16, tokens=1500)
    B, N = q.shape[:2]
    dev = "cuda"
    g = torch.Generator().manual_seed(23)
    table = torch.randn(3, 5, generator=g).to(dev).requires_grad_()
    qv = (torch.arange(N) * 3 // N).to(dev)
    sv = (torch.arange(N) % 5).to(dev)
    qd, kd, wd = (x.to(dev).requires_grad_() for x in (q, k, w))
    idx, sc = sti.sparse_topk_indexer_func(qd, kd, wd, None, 256, 0.125, 256, 0,
                                           view_bias_data=dict(q_view_ids=qv, s_view_ids=sv, view_bias=table))
    gs = torch.randn(sc.shape, generator=g).bfloat16()
    (sc.float() * gs.float().to(dev)).sum().backward()
    want = oidx.view_bias_grad(idx.cpu(), gs, qv.cpu().expand(B, N), sv.cpu().expand(B, N), (B, 3, 5)).sum(0)
    torch.testing.assert_close(table.grad.cpu(), want, atol=2e-2, rtol=1e-2)
    dq, dk, dw = sti.indexer_topk_backward(q.to(dev), k.to(dev), w.to(dev), idx, gs.to(dev), 0.125)
    assert torch.equal(qd.grad, dq) and torch.equal(kd.grad, dk) and torch.equal(wd.grad, dw)


@pytest.mark.parametrize("views", [16])
def test_full_size_sampled_rows(gpu_device, views):
    # Config C2 size (N = 21984): exact check on 384 random rows + global properties.
    q, k, w = workloads.indexer_inputs(views, 1, torch.bfloat16)
    n = q.shape[1]
    idx, sc = _gpu_topk(q, k, w, 1024)
    assert int(idx.min()) >= 0 and int(idx.max()) < n
    srt = idx[0].long().sort(-1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all()), "duplicate index in a row"
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(views))[:384]
    _check(q, k, w, idx, sc, 1024, rows=rows)


def test_long_context_s64_sampled_rows(gpu_device):
    # Config C3 size (N = 87936, the 4096-key sample path): exact check on 192 random
    # rows, plus in-range / distinct indices on every row.
    q, k, w = workloads.indexer_inputs(64, 1, torch.bfloat16)
    n = q.shape[1]
    idx, sc = _gpu_topk(q, k, w, 1024)
    assert int(idx.min()) >= 0 and int(idx.max()) < n
    srt = idx[0].long().sort(-1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all()), "duplicate index in a row"
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(64))[:192]
    _check(q, k, w, idx, sc, 1024, rows=rows)


def test_massive_ties_and_zero_scores_stay_exact(gpu_device):
    # Degenerate inputs like those of deep random-weight stacks: keys that repeat (ties in
    # the thousands) and queries whose scores are zero for almost every key (relu of
    # negative products). Such rows overflow the candidate lists or miss the sampled
    # threshold and must take the exact path; every index set must hold up to the ties.
    g = torch.Generator().manual_seed(41)
    T, S, topk = 600, 9000, 1024
    base = torch.randn(50, 4, 64, generator=g)
    k = base[torch.randint(0, 50, (S,), generator=g)].unsqueeze(0)       # 50 distinct keys
    q = torch.randn(1, T, 4, 64, generator=g)
    q[0, :200] = -k[0, :200].mean(0).sign() * k[0].abs().mean(0)          # mostly zero scores
    w = torch.ones(1, S, 4)
    q, k, w = q.bfloat16(), k.bfloat16(), w.bfloat16()
    idx, sc = _gpu_topk(q, k, w, topk)
    _check(q, k, w, idx, sc, topk)


def test_sample_defeating_scores_take_the_matrix_core_fallback(gpu_device):
    # Scores built to defeat the strided threshold sample: the 2,048 sample keys (key
    # floor(i S / 2048)) carry a component along every query's direction, the other keys
    # none, so the sampled tau (rank 81 of the sample) sits far above the true 1,024th score
    # and every row ends with too few candidates. 1,024 rows: the first 512 of the queue are
    # scored on the matrix cores, the rest by the fallback kernel itself; all exact.
    g = torch.Generator().manual_seed(61)
    T, S, topk = 1024, 43968, 1024
    d = torch.randn(4, 64, generator=g)
    q = (torch.randn(1, T, 4, 64, generator=g) * 0.3 + d).bfloat16()
    k = torch.randn(1, S, 4, 64, generator=g)
    samp = (torch.arange(2048) * S) // 2048
    k[0, samp] += 2.0 * d
    k = k.bfloat16()
    w = torch.ones(1, S, 4).bfloat16()
    idx, sc = _gpu_topk(q, k, w, topk)
    _check(q, k, w, idx, sc, topk)


def test_fallback_queues_per_batch_element(gpu_device):
    # B = 2 with every row queued (PLUS_INF): 600 rows per batch element, 512 scored on the
    # matrix cores and 88 by the fallback kernel, the two batch elements' keys kept apart.
    q, k, w = workloads.indexer_inputs(4, 2, torch.bfloat16)
    q = q[:, :600].contiguous()
    idx, sc = _gpu_topk(q, k, w, 1024, flags=sti.FLAG_TAU_PLUS_INF)
    _check(q, k, w, idx, sc, 1024)
