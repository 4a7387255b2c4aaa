"""GPU checks of head dims the kernels are not built for, which the drop-ins run on inputs
zero-padded to a built size (attention: any d <= 128 on 64 or 128; indexer: any Di <= 64 on
64), against the oracle: attention forward (o, attn_sum, lse) and backward in both layouts,
the indexer's top-k (tie-aware) and its backward. The reference's kernels take any head
dim up to these bounds (sparse_index_flash_attn.py:2034; sparse_topk_indexer.py:777,1143).
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
