"""GPU checks of head dims and indexer head counts the kernels are not built for, which the
drop-ins run on inputs zero-padded to a built size (attention: any d <= 128 on 64 or 128;
indexer: any Di <= 64 on 64, and 3, 5, 6 or 7 heads on 4 or 8 with zero heads appended),
against the oracle: attention forward (o, attn_sum, lse) and backward in both layouts, the
indexer's top-k (tie-aware) and its backward. The reference's kernels take any head dim up
to these bounds and any head count (sparse_index_flash_attn.py:2034; sparse_topk_indexer.py:
777,1009,1029,1143).
"""
import pytest
import torch

from geoweave_amd import workloads
from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa
from geoweave_amd.custom_indexer import sparse_topk_indexer_func
from oracle import attention as oatt
from oracle import indexer as oidx
from oracle.topk_check import check_topk_rows

pytestmark = pytest.mark.gpu
TOL = dict(atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("d,layout", [(32, "bthd"), (48, "bthd"), (96, "bthd"), (80, "bhtd"), (8, "bthd")])
def test_attention_padded_head_dims(gpu_device, d, layout):
    g = torch.Generator().manual_seed(d)
    B, T, S, H, K = 2, 130, 400, 4, 37
    q = torch.randn(B, T, H, d, generator=g).bfloat16()
    k = torch.randn(B, S, H, d, generator=g).bfloat16()
    v = torch.randn(B, S, H, d, generator=g).bfloat16()
    pos = workloads.random_positions(B, T, S, K, seed=d, invalid_fraction=0.2)
    do = torch.randn(B, T, H, d, generator=g).bfloat16()
    print(f"[head dims] attention d={d} {layout}", flush=True)
    qd, kd, vd = (x.cuda().requires_grad_() for x in (q, k, v))
    if layout == "bthd":
        o, attn = sifa.sparse_index_flash_attn_func(qd, kd, vd, pos.cuda())
        o.backward(do.cuda())
        got_o = o.float().cpu()
    else:
        qt, kt, vt = (x.transpose(1, 2) for x in (qd, kd, vd))
        o, attn = sifa.sparse_index_flash_attn_bhtd_func(qt, kt, vt, pos.cuda())
        assert o.shape == (B, H, T, d)
        o.backward(do.cuda().transpose(1, 2))
        got_o = o.transpose(1, 2).float().cpu()
    torch.cuda.synchronize()
    assert got_o.shape == (B, T, H, d)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos)  # default scale 1/sqrt(d) of the real d
    torch.testing.assert_close(got_o, ro, **TOL)
    torch.testing.assert_close(attn.cpu(), ra, atol=1e-4, rtol=1e-3)
    rq, rk, rv = oatt.sparse_attention_bwd(q, k, v, pos, ro.to(q.dtype), rl, do, None)
    for got, ref in ((qd.grad, rq), (kd.grad, rk), (vd.grad, rv)):
        assert got.shape == ref.shape
        torch.testing.assert_close(got.float().cpu(), ref, **TOL)


@pytest.mark.parametrize("di", [32, 16])
def test_indexer_padded_head_dims(gpu_device, di):
    g = torch.Generator().manual_seed(100 + di)
    B, T, S, Hi, K = 1, 300, 900, 4, 64
    q = torch.randn(B, T, Hi, di, generator=g).bfloat16()
    k = torch.randn(B, S, Hi, di, generator=g).bfloat16()
    w = torch.randn(B, S, Hi, generator=g).bfloat16()
    print(f"[head dims] indexer Di={di}", flush=True)
    qd, kd, wd = (x.cuda().requires_grad_() for x in (q, k, w))
    idx, sc = sparse_topk_indexer_func(qd, kd, wd, None, K, None, 256)
    torch.cuda.synchronize()
    ref = oidx.indexer_scores(q, k, w, None, None)  # default scale 1/sqrt(Di) of the real Di
    rep = check_topk_rows(ref[0], idx[0].cpu(), K)
    assert rep.ok, rep
    torch.testing.assert_close(sc.float().cpu(), ref[0].gather(1, idx[0].cpu().long()).unsqueeze(0), **TOL)
    gs = torch.randn(B, T, K, generator=g).bfloat16()
    sc.backward(gs.cuda())
    torch.cuda.synchronize()
    rq, rk, rw = oidx.indexer_topk_bwd(q, k, w, idx.cpu().long(), gs.float(), None)
    for got, ref_g in ((qd.grad, rq), (kd.grad, rk), (wd.grad, rw)):
        assert got.shape == ref_g.shape
        bad = ~torch.isclose(got.float().cpu(), ref_g, **TOL)
        assert bad.float().mean() <= 1e-3, f"{int(bad.sum())} of {bad.numel()} outside tolerance"


@pytest.mark.parametrize("heads,dtype", [(3, torch.bfloat16), (5, torch.bfloat16), (6, torch.float16),
                                         (7, torch.bfloat16), (3, torch.float32)])
def test_indexer_padded_head_counts(gpu_device, heads, dtype):
    # Zero heads appended (q = k = w = 0) add w relu(0) = 0 to every score. Top-k on random
    # inputs (tie-aware; scores at 2e-2, 1e-4 in float32), then the backward through autograd
    # on dyadic inputs, whose z are exact, against the oracle on the GPU's indices.
    g = torch.Generator().manual_seed(200 + heads)
    B, T, S, K = 2, 400, 1100, 96
    tol = dict(atol=1e-4, rtol=1e-4) if dtype == torch.float32 else TOL
    q = torch.randn(B, T, heads, 64, generator=g).to(dtype)
    k = torch.randn(B, S, heads, 64, generator=g).to(dtype)
    w = torch.randn(B, S, heads, generator=g).to(dtype)
    print(f"[head counts] indexer Hi={heads} {dtype}", flush=True)
    idx, sc = sparse_topk_indexer_func(q.cuda(), k.cuda(), w.cuda(), None, K, 0.125, 256)
    torch.cuda.synchronize()
    assert idx.shape == (B, T, K) and sc.dtype == dtype
    for b in range(B):
        ref = oidx.indexer_scores(q[b:b + 1], k[b:b + 1], w[b:b + 1], None, 0.125)[0]
        rep = check_topk_rows(ref, idx[b].cpu(), K)
        assert rep.ok, f"batch {b}: {rep}"
        torch.testing.assert_close(sc[b].float().cpu(), ref.gather(1, idx[b].cpu().long()), **tol)

    vals = torch.tensor([-1.0, -0.5, 0.0, 0.5, 1.0])
    q, k = (vals[torch.randint(0, 5, (B, n, heads, 64), generator=g)].to(dtype) for n in (T, S))
    w = torch.tensor([-0.5, 0.75, 1.0, 1.25])[torch.randint(0, 4, (B, S, heads), generator=g)].to(dtype)
    qd, kd, wd = (x.cuda().requires_grad_() for x in (q, k, w))
    idx, sc = sparse_topk_indexer_func(qd, kd, wd, None, K, 0.125, 256)
    gs = torch.randn(B, T, K, generator=g).to(dtype)
    sc.backward(gs.cuda())
    torch.cuda.synchronize()
    rq, rk, rw = oidx.indexer_topk_bwd(q, k, w, idx.cpu().long(), gs.float(), 0.125)
    for got, ref_g in ((qd.grad, rq), (kd.grad, rk), (wd.grad, rw)):
        assert got.shape == ref_g.shape and got.dtype == dtype
        torch.testing.assert_close(got.float().cpu(), ref_g, **tol)
