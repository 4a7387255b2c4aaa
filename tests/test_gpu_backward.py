"""GPU parity of the backward passes (sparse attention and indexer top-k) against the fp32
CPU oracle.

Bar: gradients within 2e-2 abs/rel in bf16/fp16 (the parity bar of this path); the
reference's own fp16 kernel check uses 1e-2 for gradients (geoweave/kernels.py:41) and is
run at that tolerance on its own shape. The backward has no float atomics, so results
are also checked to be bitwise reproducible.
"""
import pytest
import torch

from geoweave_amd import _csr, workloads
from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa
from geoweave_amd.custom_flash_attn._backward import sparse_attn_backward
from geoweave_amd.custom_indexer import sparse_topk_indexer as sti
from geoweave_amd.custom_indexer._backward import indexer_topk_backward
from oracle import attention as oatt
from oracle import indexer as oidx

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)


def _attn_grads(q, k, v, pos, do, dattn=None, scale=None, layout="bthd", dev="cuda"):
    """Forward + backward through the HIP kernels; returns CPU fp32 (dq, dk, dv) in bthd."""
    qd, kd, vd, pd, dod = (x.to(dev) for x in (q, k, v, pos, do))
    if layout == "bhtd":
        qd, kd, vd, dod = (x.transpose(1, 2).contiguous() for x in (qd, kd, vd, dod))
    o, _, lse, sc = sifa._flash_attn_forward(qd, kd, vd, pd, softmax_scale=scale, return_attn=False,
                                             q_layout=layout)
    da = None if dattn is None else dattn.to(dev)
    dq, dk, dv = sparse_attn_backward(dod, qd, kd, vd, pd, o, lse, da, sc, layout)
    torch.cuda.synchronize()
    out = [dq, dk, dv]
    if layout == "bhtd":
        out = [x.transpose(1, 2) for x in out]
    return [x.float().cpu() for x in out], o.cpu(), lse.cpu()


def _oracle_grads(q, k, v, pos, do, dattn=None, scale=None):
    o, _, lse = oatt.sparse_attention(q, k, v, pos, scale)
    # the oracle sees o rounded to the kernel dtype, as the reference's bwd reads the saved o
    o = o.to(q.dtype)
    da = None if dattn is None else dattn.to(q.dtype)
    return oatt.sparse_attention_bwd(q, k, v, pos, o, lse, do, da, scale)


def test_reference_kernel_check_shape_fp16(gpu_device):
    # geoweave/kernels.py:27-41: B=1, T=128, H=2, D=64, K=64 of 128, fp16; grads at 1e-2
    torch.manual_seed(123)
    q, k, v = (torch.randn(1, 128, 2, 64, dtype=torch.float16) for _ in range(3))
    pos = torch.rand(1, 128, 128).argsort(-1)[..., :64].to(torch.int32).contiguous()
    do = torch.randn(1, 128, 2, 64, dtype=torch.float16)
    (dq, dk, dv), _, _ = _attn_grads(q, k, v, pos, do)
    rq, rk, rv = _oracle_grads(q, k, v, pos, do)
    torch.testing.assert_close(dq, rq, atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(dk, rk, atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(dv, rv, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("with_dattn", [False, True])
@pytest.mark.parametrize("batch,seqlen,heads,topk", [(2, 128, 4, 64), (1, 256, 8, 128)])
def test_reference_test_cases_ragged_bf16(gpu_device, batch, seqlen, heads, topk, with_dattn):
    # tests/sparse_index_flash_attn_tests.py:453-454 with -1 padding (:37-44); the dattn case
    # is the KL-loss path (attn_sum feeds the indexer loss)
    q, k, v = workloads.attention_inputs(1, batch, torch.bfloat16, tokens=seqlen, heads=heads, seed=seqlen)
    pos = workloads.random_positions(batch, seqlen, seqlen, topk, seed=seqlen + 1, invalid_fraction=0.5)
    g = torch.Generator().manual_seed(seqlen + 2)
    do = torch.randn(batch, seqlen, heads, 64, generator=g).bfloat16()
    dattn = torch.randn(batch, seqlen, topk, generator=g) if with_dattn else None
    (dq, dk, dv), _, _ = _attn_grads(q, k, v, pos, do, dattn)
    rq, rk, rv = _oracle_grads(q, k, v, pos, do, dattn)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)


@pytest.mark.parametrize("heads,head_dim,layout", [(16, 64, "bthd"), (16, 64, "bhtd"), (3, 128, "bthd"),
                                                   (1, 64, "bthd"), (6, 128, "bhtd")])
def test_head_shapes_and_layouts(gpu_device, heads, head_dim, layout):
    q, k, v = workloads.attention_inputs(1, 2, torch.bfloat16, tokens=300, heads=heads, head_dim=head_dim, seed=heads)
    pos = workloads.random_positions(2, 300, 300, 77, seed=5, invalid_fraction=0.3)
    do = torch.randn(2, 300, heads, head_dim, generator=torch.Generator().manual_seed(1)).bfloat16()
    dattn = torch.randn(2, 300, 77, generator=torch.Generator().manual_seed(2))
    (dq, dk, dv), _, _ = _attn_grads(q, k, v, pos, do, dattn, scale=0.1, layout=layout)
    rq, rk, rv = _oracle_grads(q, k, v, pos, do, dattn, scale=0.1)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)


def test_hub_keys_long_lists_and_masking(gpu_device):
    # Key 0 is chosen by every query (6000 entries: the long-list sort and several work
    # items), key 1 by every other query (3000 entries: two items), and some rows hold
    # duplicates, invalid entries or nothing valid at all.
    T, H, K = 6000, 16, 32
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=T, seed=77)
    pos = workloads.random_positions(1, T, T, K, seed=78)
    pos[0, :, 0] = 0
    pos[0, ::2, 1] = 1
    pos[0, 5, :] = -1
    pos[0, 6, 3:] = T
    pos[0, 7, :] = 9  # duplicates are independent entries
    g = torch.Generator().manual_seed(79)
    do = torch.randn(1, T, H, 64, generator=g).bfloat16()
    (dq, dk, dv), _, _ = _attn_grads(q, k, v, pos, do)
    rq, rk, rv = _oracle_grads(q, k, v, pos, do)
    assert torch.all(dq[0, 5] == 0)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)
    # keys never selected get exactly zero
    chosen = torch.zeros(T, dtype=torch.bool)
    valid = (pos[0] >= 0) & (pos[0] < T)
    chosen[pos[0][valid].long()] = True
    assert torch.all(dk[0, ~chosen] == 0) and torch.all(dv[0, ~chosen] == 0)


def test_backward_is_bitwise_reproducible(gpu_device):
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=5000, seed=90)
    pos = workloads.random_positions(1, 5000, 5000, 256, seed=91)
    pos[0, :, 0] = 3  # one list longer than the in-LDS sort
    do = torch.randn(1, 5000, 16, 64, generator=torch.Generator().manual_seed(92)).bfloat16()
    dattn = torch.randn(1, 5000, 256, generator=torch.Generator().manual_seed(93))
    a, _, _ = _attn_grads(q, k, v, pos, do, dattn)
    _csr.clear_cache()
    b, _, _ = _attn_grads(q, k, v, pos, do, dattn)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_autograd_function_matches_oracle(gpu_device):
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=512, seed=21)
    pos = workloads.random_positions(1, 512, 512, 128, seed=22)
    g = torch.Generator().manual_seed(23)
    do = torch.randn(1, 512, 16, 64, generator=g).bfloat16()
    dattn = torch.randn(1, 512, 128, generator=g)
    qd, kd, vd = (x.cuda().requires_grad_() for x in (q, k, v))
    o, attn = sifa.sparse_index_flash_attn_func(qd, kd, vd, pos.cuda())
    ((o.float() * do.cuda().float()).sum() + (attn * dattn.cuda()).sum()).backward()
    rq, rk, rv = _oracle_grads(q, k, v, pos, do, dattn)
    torch.testing.assert_close(qd.grad.float().cpu(), rq, **TOL)
    torch.testing.assert_close(kd.grad.float().cpu(), rk, **TOL)
    torch.testing.assert_close(vd.grad.float().cpu(), rv, **TOL)


def test_training_shape_sampled(gpu_device):
    # Config C4 (B=2, S=24 views, N=32976, H=16, D=64, K=1024): dq on sampled query rows,
    # dk/dv on sampled keys (incl. the most-selected key), plus the exact invariants
    # sum_s dV = sum_t dO and sum_s dK = 0 per head on all rows.
    views, B, K = 24, 2, 1024
    q, k, v = workloads.attention_inputs(views, B, torch.bfloat16)
    n = q.shape[1]
    g = torch.Generator().manual_seed(views)
    # distinct positions per row (as top-k gives), with one key listed by every query, so
    # the forward takes the masked dense pass and the CSR holds a key longer than a work item
    pos = workloads.distinct_positions(B, n, n, K, seed=views, hub=12345)
    pos[1, 100:140, 5] = pos[1, 100:140, 6]  # repeats in a few rows: those blocks gather
    do = torch.randn(B, n, 16, 64, generator=g).bfloat16()
    (dq, dk, dv), o, lse = _attn_grads(q, k, v, pos, do)
    rows = torch.cat([torch.arange(100, 140, 8), torch.randperm(n, generator=g)[:96]])
    _, _, rlse = oatt.sparse_attention(q[:, rows], k, v, pos[:, rows])
    torch.testing.assert_close(lse[:, rows], rlse, atol=1e-4, rtol=1e-4)
    rq, _, _ = oatt.sparse_attention_bwd(q[:, rows], k, v, pos[:, rows], o[:, rows], lse[:, rows], do[:, rows])
    torch.testing.assert_close(dq[:, rows], rq, **TOL)
    counts = torch.bincount(pos[0].reshape(-1).long(), minlength=n)
    keys = torch.cat([counts.argmax().view(1), torch.randperm(n, generator=g)[:15]])
    rk, rv = oatt.sparse_attention_bwd_keys(q, k, v, pos, o, lse, do, keys)
    torch.testing.assert_close(dk[:, keys], rk, **TOL)
    torch.testing.assert_close(dv[:, keys], rv, **TOL)
    torch.testing.assert_close(dv.sum(1), do.float().sum(1), atol=0.5, rtol=1e-2)
    assert dk.sum(1).abs().max() < 0.5


# ----------------------------------------------------------------------------- indexer


def _dyadic(shape, g, vals=(-1.0, -0.5, 0.0, 0.5, 1.0)):
    """Values whose dot products over 64 dims are exact in fp32 in any order."""
    t = torch.tensor(vals)
    return t[torch.randint(0, len(vals), shape, generator=g)]


def _idx_grads(q, k, w, idx, grad, scale=0.125, dev="cuda"):
    dq, dk, dw = indexer_topk_backward(q.to(dev), k.to(dev), w.to(dev), idx.to(dev), grad.to(dev), scale)
    torch.cuda.synchronize()
    return dq.float().cpu(), dk.float().cpu(), dw.float().cpu()


@pytest.mark.parametrize("heads", [1, 2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_indexer_bwd_exact_dot_products(gpu_device, heads, dtype):
    # Dyadic q/k make every z exact, so the relu decisions match the oracle's bit for bit
    # and only fp32 accumulation order differs.
    g = torch.Generator().manual_seed(heads)
    B, T, S, K = 2, 700, 900, 96
    q = _dyadic((B, T, heads, 64), g).to(dtype)
    k = _dyadic((B, S, heads, 64), g).to(dtype)
    w = _dyadic((B, S, heads), g, (-0.5, 0.75, 1.0, 1.25, 1.5)).to(dtype)
    idx = torch.stack([workloads.random_positions(1, T, S, K, seed=heads * 10 + b)[0] for b in range(B)])
    idx[0, :, 0] = 5  # a key chosen by every query
    grad = torch.randn(B, T, K, generator=g).to(dtype)
    dq, dk, dw = _idx_grads(q, k, w, idx, grad)
    rq, rk, rw = oidx.indexer_topk_bwd(q, k, w, idx, grad, 0.125)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dw, rw, **TOL)


def test_indexer_autograd_through_topk(gpu_device):
    # End to end: forward top-k on the GPU, backward through the selected scores; the
    # oracle differentiates scores.gather(idx) (indexer.py:600-603) on the same indices.
    g = torch.Generator().manual_seed(5)
    q = _dyadic((1, 1000, 4, 64), g).bfloat16()
    k = _dyadic((1, 1000, 4, 64), g).bfloat16()
    w = _dyadic((1, 1000, 4), g, (0.5, 0.75, 1.0, 1.25)).bfloat16()
    qd, kd, wd = (x.cuda().requires_grad_() for x in (q, k, w))
    idx, sc = sti.sparse_topk_indexer_func(qd, kd, wd, None, 64, 0.125, 256)
    gs = torch.randn(sc.shape, generator=g).bfloat16()
    sc.backward(gs.cuda())
    rq, rk, rw = oidx.indexer_topk_bwd(q, k, w, idx.cpu(), gs, 0.125)
    torch.testing.assert_close(qd.grad.float().cpu(), rq, **TOL)
    torch.testing.assert_close(kd.grad.float().cpu(), rk, **TOL)
    torch.testing.assert_close(wd.grad.float().cpu(), rw, **TOL)


def test_indexer_bwd_layer_inputs_sampled(gpu_device):
    # Layer-shaped bf16 inputs (S=4 views, top-k 1024 from the HIP forward): dq on sampled
    # rows and dk/dw on sampled keys. z values within rounding of 0 may flip the relu gate
    # relative to the oracle; such entries are rare, so at most 0.1% of elements may
    # exceed the tolerance.
    q, k, w = workloads.indexer_inputs(4, 1, torch.bfloat16)
    n = q.shape[1]
    qd, kd, wd = q.cuda(), k.cuda(), w.cuda()
    idx, sc = sti.indexer_topk_forward(qd, kd, wd, None, 1024, 0.125)
    g = torch.Generator().manual_seed(4)
    grad = torch.randn(sc.shape, generator=g).bfloat16()
    dq, dk, dw = _idx_grads(q, k, w, idx.cpu(), grad)
    rows = torch.randperm(n, generator=g)[:128]
    rq, _, _ = oidx.indexer_topk_bwd(q[:, rows], k, w, idx.cpu()[:, rows], grad[:, rows], 0.125)
    keys = torch.randperm(n, generator=g)[:32]
    rk, rw = oidx.indexer_topk_bwd_keys(q, k, w, idx.cpu(), grad, keys, 0.125)
    for got, ref in ((dq[:, rows], rq), (dk[:, keys], rk), (dw[:, keys], rw)):
        bad = ~torch.isclose(got, ref, **TOL)
        assert bad.float().mean() <= 1e-3, f"{int(bad.sum())} of {bad.numel()} outside tolerance"
