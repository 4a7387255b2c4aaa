"""GPU parity of the indexer top-k and its backward with float32 q/k/w.

The reference's indexer computes in ``q.dtype`` for any float type
(``easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:1293``; the Triton block kernel
upcasts, ``:1049-1052``) and its caller casts q/k/w to ``score_dtype``, which may be float32
(``easyvolcap/official_vggt/layers/indexer.py:321-326``). Bar (float32): index sets
bit-exact except where oracle fp32 scores tie within 1e-6 relative; returned scores and
gradients within 1e-4.
"""
import json
from pathlib import Path

import pytest
import torch

from geoweave_amd import workloads
from geoweave_amd.custom_indexer import sparse_topk_indexer as sti
from geoweave_amd.custom_indexer._backward import indexer_topk_backward
from oracle import indexer as oidx
from oracle.topk_check import check_topk_rows

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL32 = dict(atol=1e-4, rtol=1e-4)
F32 = torch.float32


def _gpu_topk(q, k, w, topk, scale=0.125, mask=None, flags=0, view_bias=None, dev="cuda"):
    m = None if mask is None else mask.to(dev)
    vb = None if view_bias is None else tuple(x.to(dev) for x in view_bias)
    idx, sc = sti.indexer_topk_forward(q.to(dev), k.to(dev), w.to(dev), m, topk, scale, flags, view_bias=vb)
    torch.cuda.synchronize()
    assert sc.dtype == F32
    return idx.cpu(), sc.cpu()


def _check_all_rows(q, k, w, idx, sc, topk, scale=0.125, mask=None, view_bias=None):
    for b in range(q.shape[0]):
        mb = None if mask is None else mask[b:b + 1]
        vb = None if view_bias is None else tuple(x[b:b + 1] for x in view_bias)
        ref = oidx.indexer_scores(q[b:b + 1], k[b:b + 1], w[b:b + 1], mb, scale, view_bias=vb)[0]
        rep = check_topk_rows(ref, idx[b], topk)
        assert rep.ok, f"batch {b}: {rep}"
        torch.testing.assert_close(sc[b], ref.gather(1, idx[b].long()), **TOL32)
    return rep


def test_c1_every_row_fp32(gpu_device):
    # Config C1 (S = 4 views, N = 5,496, 4 x 64 heads, top-k 1024) in float32, the
    # reference's own CPU configuration: every row, through the sampled threshold.
    q, k, w = workloads.indexer_inputs(4, 1, F32)
    idx, sc = _gpu_topk(q, k, w, 1024)
    assert idx.shape == (1, q.shape[1], 1024) and idx.dtype == torch.int32
    rep = _check_all_rows(q, k, w, idx, sc, 1024)
    print(f"C1 fp32: exact rows {rep.rows_exact}/{rep.rows}, tie-swapped {rep.rows_tie_swapped}")


@pytest.mark.parametrize("case", json.loads((GOLDEN / "indexer_kat.json").read_text()), ids=lambda c: c["name"])
def test_golden_kat_fp32(gpu_device, case):
    q = torch.nn.functional.pad(torch.tensor(case["q"]).unsqueeze(0), (0, 64 - len(case["q"][0][0])))
    k = torch.nn.functional.pad(torch.tensor(case["k"]).unsqueeze(0), (0, 64 - len(case["k"][0][0])))
    w = torch.tensor(case["w"]).unsqueeze(0)
    mask = None if case["mask"] is None else torch.tensor(case["mask"]).unsqueeze(0)
    idx, sc = _gpu_topk(q, k, w, case["topk"], case["scale"], mask)
    ref = torch.tensor(case["scores"], dtype=F32)
    rep = check_topk_rows(ref, idx[0], case["topk"])
    assert rep.ok, rep
    torch.testing.assert_close(sc[0], ref.gather(1, idx[0].long()), **TOL32)
    if case["name"].startswith("reference"):
        assert [sorted(r) for r in idx[0].tolist()] == case["expected_sets"]


@pytest.mark.parametrize("case", json.loads((GOLDEN / "indexer_view_bias_kat.json").read_text()),
                         ids=lambda c: c["name"])
def test_view_bias_golden_kat_fp32(gpu_device, case):
    dev = "cuda"
    pad = lambda x: torch.nn.functional.pad(x, (0, 64 - x.shape[-1]))  # noqa: E731
    q = pad(torch.tensor(case["q"]).unsqueeze(0)).to(dev).requires_grad_()
    k = pad(torch.tensor(case["k"]).unsqueeze(0)).to(dev).requires_grad_()
    w = torch.tensor(case["w"]).unsqueeze(0).to(dev).requires_grad_()
    mask = None if case["mask"] is None else torch.tensor(case["mask"]).unsqueeze(0).to(dev)
    table = torch.tensor(case["view_bias"], device=dev, requires_grad=True)
    vbd = dict(q_view_ids=torch.tensor(case["q_view_ids"], device=dev),
               s_view_ids=torch.tensor(case["s_view_ids"], device=dev), view_bias=table)
    idx, sc = sti.sparse_topk_indexer_func(q, k, w, mask, case["topk"], case["scale"], 256, 0, view_bias_data=vbd)
    assert sc.dtype == F32
    ref = torch.tensor(case["scores"], dtype=F32)
    rep = check_topk_rows(ref, idx[0].cpu(), case["topk"])
    assert rep.ok, rep
    torch.testing.assert_close(sc[0].cpu(), ref.gather(1, idx[0].long().cpu()), **TOL32)
    if "table_grad_of_sum" in case:
        sc.sum().backward()
        torch.testing.assert_close(table.grad.cpu(), torch.tensor(case["table_grad_of_sum"]), atol=0, rtol=0)


def test_mask_and_view_bias_fp32(gpu_device):
    # B = 2 of 2,000 tokens: an additive mask with -inf entries and a view-bias table, both
    # in float32.
    q, k, w = workloads.indexer_inputs(1, 2, F32, tokens=2000)
    B, N = q.shape[:2]
    g = torch.Generator().manual_seed(31)
    mask = torch.randn(B, N, N, generator=g)
    mask[torch.rand(B, N, N, generator=g) < 0.1] = float("-inf")
    table = 2 * torch.randn(B, 4, 4, generator=g)
    qv = (torch.arange(N) // 500).expand(B, N).contiguous()
    sv = (torch.arange(N) // 500).flip(0).expand(B, N).contiguous()
    vb = (qv.to(torch.int32), sv.to(torch.int32), table)
    idx, sc = _gpu_topk(q, k, w, 512, mask=mask, view_bias=vb)
    _check_all_rows(q, k, w, idx, sc, 512, mask=mask, view_bias=(qv, sv, table))


@pytest.mark.parametrize("heads", [1, 2])
def test_other_head_counts_fp32(gpu_device, heads):
    g = torch.Generator().manual_seed(100 + heads)
    n = 5000
    q = torch.randn(1, n, heads, 64, generator=g)
    k = torch.randn(1, n, heads, 64, generator=g)
    w = 1 + 0.3 * torch.randn(1, n, heads, generator=g)
    idx, sc = _gpu_topk(q, k, w, 300)
    _check_all_rows(q, k, w, idx, sc, 300)


def test_full_rows_path_fp32(gpu_device):
    # k = 9,000 of 9,500 keys: every row scored over every key on the matrix cores (fp32
    # products) and selected exactly, in two rounds of rows.
    g = torch.Generator().manual_seed(31)
    q = torch.randn(1, 600, 4, 64, generator=g)
    k = torch.randn(1, 9500, 4, 64, generator=g)
    w = 1 + 0.3 * torch.randn(1, 9500, 4, generator=g)
    idx, sc = _gpu_topk(q, k, w, 9000)
    _check_all_rows(q, k, w, idx, sc, 9000)


def test_eight_heads_fp32_not_built(gpu_device):
    q = torch.zeros(1, 8, 8, 64, device="cuda")
    w = torch.zeros(1, 8, 8, device="cuda")
    with pytest.raises(NotImplementedError, match="float32"):
        sti.indexer_topk_forward(q, q, w, None, 4, 0.125)


@pytest.mark.parametrize("flags,tokens", [(sti.FLAG_TAU_PLUS_INF, None), (sti.FLAG_TAU_MINUS_INF, 12000),
                                          (sti.FLAG_FORCE_WIDE, None), (sti.FLAG_FORCE_WIDE, 2000)])
def test_forced_fallback_paths_fp32(gpu_device, flags, tokens):
    # The brute-force kernel (every query, or overflowed lists at N = 12,000) and the LDS
    # select path (with and without the sampled threshold) in float32.
    q, k, w = workloads.indexer_inputs(4, 1, F32, tokens=tokens)
    q = q[:, :768].contiguous()
    idx, sc = _gpu_topk(q, k, w, 1024, flags=flags)
    _check_all_rows(q, k, w, idx, sc, 1024)


def _dyadic(shape, g, vals=(-1.0, -0.5, 0.0, 0.5, 1.0)):
    """Values whose dot products over 64 dims are exact in fp32 in any order."""
    t = torch.tensor(vals)
    return t[torch.randint(0, len(vals), shape, generator=g)]


@pytest.mark.parametrize("heads", [1, 2, 4])
def test_indexer_bwd_exact_dot_products_fp32(gpu_device, heads):
    # Dyadic q/k/w: every z is exact, so the relu decisions equal the oracle's; float32
    # gradients against the oracle's at 1e-4 (only the fp32 accumulation order differs).
    g = torch.Generator().manual_seed(200 + heads)
    B, T, S, K = 2, 700, 900, 96
    q = _dyadic((B, T, heads, 64), g)
    k = _dyadic((B, S, heads, 64), g)
    w = _dyadic((B, S, heads), g, (-0.5, 0.75, 1.0, 1.25, 1.5))
    idx = torch.stack([workloads.random_positions(1, T, S, K, seed=heads * 10 + b)[0] for b in range(B)])
    idx[0, :, 0] = 5  # a key chosen by every query
    grad = torch.randn(B, T, K, generator=g)
    dev = "cuda"
    dq, dk, dw = indexer_topk_backward(q.to(dev), k.to(dev), w.to(dev), idx.to(dev), grad.to(dev), 0.125)
    assert dq.dtype == dk.dtype == dw.dtype == F32
    rq, rk, rw = oidx.indexer_topk_bwd(q, k, w, idx, grad, 0.125)
    torch.testing.assert_close(dq.cpu(), rq, **TOL32)
    torch.testing.assert_close(dk.cpu(), rk, **TOL32)
    torch.testing.assert_close(dw.cpu(), rw, **TOL32)


def test_autograd_layer_inputs_fp32(gpu_device):
    # C1-shaped float32 inputs through the drop-in with autograd: the top-k indices from the
    # GPU, the gradients of the selected scores against the oracle on sampled rows and keys
    # (including the most-selected key). A z within rounding of 0 may flip the relu gate
    # relative to the oracle: at most 0.1 % of elements may exceed the tolerance.
    q, k, w = workloads.indexer_inputs(4, 1, F32)
    n = q.shape[1]
    dev = "cuda"
    qd, kd, wd = (x.to(dev).requires_grad_() for x in (q, k, w))
    idx, sc = sti.sparse_topk_indexer_func(qd, kd, wd, None, 1024, 0.125, 256)
    g = torch.Generator().manual_seed(7)
    gs = torch.randn(sc.shape, generator=g)
    sc.backward(gs.to(dev))
    idx_c = idx.cpu()
    rows = torch.randperm(n, generator=g)[:128]
    rq, _, _ = oidx.indexer_topk_bwd(q[:, rows], k, w, idx_c[:, rows], gs[:, rows], 0.125)
    counts = torch.bincount(idx_c.flatten().long(), minlength=n)
    keys = torch.cat([counts.argmax().view(1), torch.randperm(n, generator=g)[:31]])
    rk, rw = oidx.indexer_topk_bwd_keys(q, k, w, idx_c, gs, keys, 0.125)
    for got, ref in ((qd.grad.cpu()[:, rows], rq), (kd.grad.cpu()[:, keys], rk), (wd.grad.cpu()[:, keys], rw)):
        bad = ~torch.isclose(got, ref, **TOL32)
        assert bad.float().mean() <= 1e-3, f"{int(bad.sum())} of {bad.numel()} outside tolerance"
