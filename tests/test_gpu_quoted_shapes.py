"""GPU parity at the shapes the measurements are quoted on.

* Metric row (S = 32 views, N = 43,968): the bench's own inputs and calls (indexer top-k,
  then the inference attention forward, which takes the masked dense pass); index sets on
  sampled rows (tie-aware), o and lse on sampled rows.
* C1 (S = 4, N = 5,496, K = 1,024, H = 16): every row — indices, then o, lse and attn_sum
  of the attention over the indexer's own selection.
* C4 (B = 2, S = 24, N = 32,976): the indexer's own indices (both batch elements, sampled
  rows), the training forward over them (dense pass + attn_sum: o, attn_sum, lse on sampled
  rows) and the attention backward (dq on sampled rows, dk/dv on sampled keys, the exact
  invariants on all).
* C5 (the aggregator at S = 32, 518 x 518 images): the first and last sparse layers' inputs
  captured inside the forward; indices and attention output on sampled rows.

Bar: index sets bit-exact except inside the 1e-6 relative tie window (oracle/topk_check.py);
o and gradients 2e-2 abs/rel (bf16), lse 1e-4, attn_sum 1e-4 abs / 1e-3 rel.
"""
import pytest
import torch

from geoweave_amd import aggregator as agg
from geoweave_amd import dsa_layer, workloads
from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa
from geoweave_amd.custom_flash_attn._backward import sparse_attn_backward
from geoweave_amd.custom_indexer import sparse_topk_indexer as sti
from oracle import attention as oatt
from oracle import indexer as oidx
from oracle.topk_check import check_topk_rows

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)
LSE_TOL = dict(atol=1e-4, rtol=1e-4)
ATTN_TOL = dict(atol=1e-4, rtol=1e-3)


def _check_indices(q, k, w, idx, sc, topk, rows, scale=0.125):
    """Tie-aware set check of every batch element on the given rows (CPU tensors), plus the
    returned scores, plus in-range and distinct indices on every row."""
    n = k.shape[1]
    assert int(idx.min()) >= 0 and int(idx.max()) < n
    srt = idx.long().sort(-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all()), "duplicate index in a row"
    for b in range(q.shape[0]):
        ref = oidx.indexer_scores(q[b:b + 1, rows], k[b:b + 1], w[b:b + 1], None, scale)[0]
        rep = check_topk_rows(ref, idx[b, rows], topk)
        assert rep.ok, f"batch {b}: {rep}"
        torch.testing.assert_close(sc[b, rows].float(), ref.gather(1, idx[b, rows].long()), **TOL)


def test_metric_row_s32_indices_and_attention(gpu_device):
    views = 32
    lay = workloads.layer_inputs(views, 1, torch.bfloat16)
    n = lay.tokens
    print(f"[metric row] S={views} N={n}", flush=True)
    qi, ki, wi, q, k, v = (x.cuda() for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v))
    # the bench's calls (bench.py: one step)
    idx, sc = sti.sparse_topk_indexer_inference_func(qi, ki, wi, qi.new_empty(0), 1024, 0.125, 256, 0,
                                                     return_scores=True)
    assert sifa._use_dense(n, 1024, 16, 64, 0.125), "the metric row runs the masked dense pass"
    o, _, lse, _ = sifa._flash_attn_forward(q, k, v, idx, softmax_scale=0.125, return_attn=False)
    o_inf, _ = sifa.sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=0.125)
    torch.cuda.synchronize()
    assert torch.equal(o, o_inf)
    idx, sc, o, lse = idx.cpu(), sc.cpu(), o.float().cpu(), lse.cpu()
    g = torch.Generator().manual_seed(views)
    rows = torch.randperm(n, generator=g)[:256]
    _check_indices(lay.q_idx, lay.k_idx, lay.w_idx, idx, sc, 1024, rows)
    rows = rows[:128]
    ro, _, rl = oatt.sparse_attention(lay.q[:, rows], lay.k, lay.v, idx[:, rows], 0.125)
    torch.testing.assert_close(o[:, rows], ro, **TOL)
    torch.testing.assert_close(lse[:, rows], rl, **LSE_TOL)


def test_c1_every_row(gpu_device):
    views = 4
    lay = workloads.layer_inputs(views, 1, torch.bfloat16)
    n = lay.tokens
    print(f"[C1] S={views} N={n}", flush=True)
    qi, ki, wi, q, k, v = (x.cuda() for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v))
    idx, sc = sti.sparse_topk_indexer_func(qi, ki, wi, qi.new_empty(0), 1024, 0.125, 256, 0)
    o, attn, lse, _ = sifa._flash_attn_forward(q, k, v, idx, softmax_scale=0.125, return_attn=True)
    o_inf, _ = sifa.sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=0.125)
    torch.cuda.synchronize()
    assert torch.equal(o, o_inf), "attn_sum must not change o"
    idx, sc = idx.cpu(), sc.cpu()
    _check_indices(lay.q_idx, lay.k_idx, lay.w_idx, idx, sc, 1024, torch.arange(n))
    ro, ra, rl = oatt.sparse_attention(lay.q, lay.k, lay.v, idx, 0.125)
    torch.testing.assert_close(o.float().cpu(), ro, **TOL)
    torch.testing.assert_close(lse.cpu(), rl, **LSE_TOL)
    torch.testing.assert_close(attn.cpu(), ra, **ATTN_TOL)


def test_c4_indexer_indices_training_forward_and_backward(gpu_device):
    views, B = 24, 2
    lay = workloads.layer_inputs(views, B, torch.bfloat16)
    n = lay.tokens
    print(f"[C4] B={B} S={views} N={n}", flush=True)
    qi, ki, wi, q, k, v = (x.cuda() for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v))
    idx, sc = sti.sparse_topk_indexer_func(qi, ki, wi, qi.new_empty(0), 1024, 0.125, 256, 0)
    assert sifa._use_dense(n, 1024, 16, 64, 0.125), "C4 runs the masked dense pass with attn_sum"
    o, attn, lse, scale = sifa._flash_attn_forward(q, k, v, idx, softmax_scale=0.125, return_attn=True)
    g = torch.Generator().manual_seed(views)
    do = torch.randn(B, n, 16, 64, generator=g).bfloat16()
    dq, dk, dv = sparse_attn_backward(do.cuda(), q, k, v, idx, o, lse, None, scale, "bthd")
    torch.cuda.synchronize()
    idx, sc = idx.cpu(), sc.cpu()
    o, attn, lse = o.cpu(), attn.cpu(), lse.cpu()
    dq, dk, dv = dq.float().cpu(), dk.float().cpu(), dv.float().cpu()
    rows = torch.randperm(n, generator=g)[:128]
    _check_indices(lay.q_idx, lay.k_idx, lay.w_idx, idx, sc, 1024, rows)
    rows = rows[:64]
    ro, ra, rl = oatt.sparse_attention(lay.q[:, rows], lay.k, lay.v, idx[:, rows], 0.125)
    torch.testing.assert_close(o[:, rows].float(), ro, **TOL)
    torch.testing.assert_close(attn[:, rows], ra, **ATTN_TOL)
    torch.testing.assert_close(lse[:, rows], rl, **LSE_TOL)
    torch.testing.assert_close(attn.sum(-1), torch.full((B, n), 16.0), atol=2e-3, rtol=1e-4)
    rq, _, _ = oatt.sparse_attention_bwd(lay.q[:, rows], lay.k, lay.v, idx[:, rows], o[:, rows], lse[:, rows],
                                         do[:, rows], None, 0.125)
    torch.testing.assert_close(dq[:, rows], rq, **TOL)
    counts = torch.bincount(idx[0].reshape(-1).long(), minlength=n)
    keys = torch.cat([counts.argmax().view(1), torch.randperm(n, generator=g)[:11]])
    rk, rv = oatt.sparse_attention_bwd_keys(lay.q, lay.k, lay.v, idx, o, lse, do, keys, 0.125)
    torch.testing.assert_close(dk[:, keys], rk, **TOL)
    torch.testing.assert_close(dv[:, keys], rv, **TOL)
    torch.testing.assert_close(dv.sum(1), do.float().sum(1), atol=0.5, rtol=1e-2)
    assert dk.sum(1).abs().max() < 0.5


def _euler_sums(x, dx, rows_dim):
    """sum over heads and dims of x * dx per row (fp32)."""
    return (x.float() * dx.float()).reshape(x.shape[0], x.shape[1], -1).sum(-1)


def test_c4_indexer_backward(gpu_device):
    # The indexer backward at C4 (B = 2, S = 24, N = 32,976) on the indexer's own indices:
    # dq on sampled rows of both batch elements and dk/dw on sampled keys (the most-selected
    # key of each element among them) against the oracle; a z within rounding of 0 may flip
    # the relu gate relative to the oracle, so at most 0.1 % of elements may exceed the
    # tolerance. Every row and key is then checked through the score's degree-1 homogeneity
    # (score = sum_h w relu(scale q.k) is linear in q, in k and in w along each ray):
    #   sum_h q[t,h].dq[t,h] = sum_j g[t,j] score[t,j]                 (every row t)
    #   sum_h k[s,h].dk[s,h] = sum_h w[s,h] dw[s,h] = sum_{idx[t,j]=s} g[t,j] score[t,j]
    views, B = 24, 2
    lay = workloads.layer_inputs(views, B, torch.bfloat16)
    n = lay.tokens
    print(f"[C4 indexer backward] B={B} S={views} N={n}", flush=True)
    qi, ki, wi = (x.cuda() for x in (lay.q_idx, lay.k_idx, lay.w_idx))
    idx, sc = sti.sparse_topk_indexer_inference_func(qi, ki, wi, qi.new_empty(0), 1024, 0.125, 256, 0)
    g = torch.Generator().manual_seed(2400)
    gs = torch.randn(B, n, 1024, generator=g).bfloat16()
    dq, dk, dw = sti.indexer_topk_backward(qi, ki, wi, idx, gs.cuda(), 0.125)
    torch.cuda.synchronize()
    idx, sc = idx.cpu(), sc.cpu()
    dq, dk, dw = dq.float().cpu(), dk.float().cpu(), dw.float().cpu()
    for b in range(B):
        rows = torch.randperm(n, generator=g)[:64]
        rq, _, _ = oidx.indexer_topk_bwd(lay.q_idx[b:b + 1, rows], lay.k_idx[b:b + 1], lay.w_idx[b:b + 1],
                                         idx[b:b + 1, rows], gs[b:b + 1, rows], 0.125)
        counts = torch.bincount(idx[b].reshape(-1).long(), minlength=n)
        keys = torch.cat([counts.argmax().view(1), torch.randperm(n, generator=g)[:15]])
        rk, rw = oidx.indexer_topk_bwd_keys(lay.q_idx[b:b + 1], lay.k_idx[b:b + 1], lay.w_idx[b:b + 1],
                                            idx[b:b + 1], gs[b:b + 1], keys, 0.125)
        for got, ref in ((dq[b:b + 1, rows], rq), (dk[b:b + 1, keys], rk), (dw[b:b + 1, keys], rw)):
            bad = ~torch.isclose(got, ref, **TOL)
            assert bad.float().mean() <= 1e-3, f"batch {b}: {int(bad.sum())} of {bad.numel()} outside tolerance"
    gsc = gs.float() * sc.float()  # [B, T, K]
    row_rhs, row_mag = gsc.sum(-1), gsc.abs().sum(-1)
    row_lhs = _euler_sums(lay.q_idx, dq, 2)
    assert bool(((row_lhs - row_rhs).abs() <= 2e-2 * row_mag + 1e-3).all()), "row identity sum q.dq"
    for b in range(B):
        flat = idx[b].reshape(-1).long()
        key_rhs = torch.zeros(n).index_add_(0, flat, gsc[b].reshape(-1))
        key_mag = torch.zeros(n).index_add_(0, flat, gsc[b].reshape(-1).abs())
        lhs_k = _euler_sums(lay.k_idx[b:b + 1], dk[b:b + 1], 2)[0]
        lhs_w = (lay.w_idx[b].float() * dw[b]).sum(-1)
        assert bool(((lhs_k - key_rhs).abs() <= 2e-2 * key_mag + 1e-3).all()), f"batch {b}: key identity k.dk"
        assert bool(((lhs_w - key_rhs).abs() <= 2e-2 * key_mag + 1e-3).all()), f"batch {b}: key identity w.dw"


def test_c5_aggregator_sparse_layers_sampled(gpu_device, monkeypatch):
    # The C5 workload of the bench (aggregator.random_init_, seeded images); the first (9)
    # and last (19) sparse layers' indexer and attention inputs are captured in the forward.
    views, topk = 32, 1024
    dev = torch.device("cuda", 0)
    with torch.device(dev):
        m = agg.Aggregator(indexer_layers="9-19", topk=topk)
    m = agg.random_init_(m, 20261201).to(torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(20261201 + views)
    images = torch.rand(1, views, 3, 518, 518, generator=g, device=dev)
    calls = {"idx": [], "attn": []}
    want = {0, 10}  # call numbers of layers 9 and 19
    real_idx = dsa_layer.sparse_topk_indexer_inference_func
    real_attn = dsa_layer.sparse_index_flash_attn_inference_func

    def spy_idx(q, k, w, *a, **kw):
        out = real_idx(q, k, w, *a, **kw)
        if len(calls["idx"]) in want:
            calls["idx"].append((q.cpu(), k.cpu(), w.cpu(), out[0].cpu()))
        else:
            calls["idx"].append(None)
        return out

    def spy_attn(q, k, v, pos, *a, **kw):
        out = real_attn(q, k, v, pos, *a, **kw)
        if len(calls["attn"]) in want:
            calls["attn"].append((q.cpu(), k.cpu(), v.cpu(), pos.cpu(), out[0].cpu(), kw.get("softmax_scale")))
        else:
            calls["attn"].append(None)
        return out

    monkeypatch.setattr(dsa_layer, "sparse_topk_indexer_inference_func", spy_idx)
    monkeypatch.setattr(dsa_layer, "sparse_index_flash_attn_inference_func", spy_attn)
    print(f"[C5] aggregator S={views}", flush=True)
    m(images)
    torch.cuda.synchronize()
    assert len(calls["idx"]) == 11 and len(calls["attn"]) == 11
    gen = torch.Generator().manual_seed(5)
    for c in sorted(want):
        qi, ki, wi, idx = calls["idx"][c]
        q, k, v, pos, o, scale = calls["attn"][c]
        assert torch.equal(pos, idx)
        n = q.shape[1]
        print(f"[C5] sparse call {c}: N={n}", flush=True)
        rows = torch.randperm(n, generator=gen)[:96]
        ref = oidx.indexer_scores(qi[:, rows], ki, wi, None, 0.125)[0]
        rep = check_topk_rows(ref, idx[0, rows], topk)
        assert rep.ok, f"call {c}: {rep}"
        ro, _, _ = oatt.sparse_attention(q[:, rows], k, v, pos[:, rows], scale)
        torch.testing.assert_close(o[:, rows].float(), ro, **TOL)
