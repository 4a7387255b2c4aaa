"""GPU parity of the masked dense attention backward (gw_sparse_attn_bwd_dense) against the
fp32 CPU oracle and against the CSR backward (gw_sparse_attn_bwd), an independent
implementation.

The dense passes serve the backward without an attn_sum gradient (the reference presets
detach the attention mass before the indexer loss, dsa_attention.py:4694-4695) when every row
lists distinct positions and every input is finite; other calls must come back through the CSR
path with the same results. Bar: 2e-2 abs/rel in bf16/fp16 (the parity bar of this path).
"""
import pytest
import torch

from geoweave_amd import workloads
from geoweave_amd.custom_flash_attn import _backward
from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa
from geoweave_amd.custom_flash_attn._backward import sparse_attn_backward
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)


def _fwd(q, k, v, pos, scale=None, layout="bthd"):
    qd, kd, vd, pd = (x.cuda() for x in (q, k, v, pos))
    if layout == "bhtd":
        qd, kd, vd = (x.transpose(1, 2).contiguous() for x in (qd, kd, vd))
    o, _, lse, sc = sifa._flash_attn_forward(qd, kd, vd, pd, softmax_scale=scale, return_attn=False,
                                             q_layout=layout)
    return qd, kd, vd, pd, o, lse, sc


def _bwd(do, qd, kd, vd, pd, o, lse, sc, layout="bthd", path="auto"):
    dod = do.cuda()
    if layout == "bhtd":
        dod = dod.transpose(1, 2).contiguous()
    old = _backward.BACKWARD_PATH
    _backward.BACKWARD_PATH = path
    try:
        dq, dk, dv = sparse_attn_backward(dod, qd, kd, vd, pd, o, lse, None, sc, layout)
    finally:
        _backward.BACKWARD_PATH = old
    torch.cuda.synchronize()
    taken = _backward.last_path
    out = [dq, dk, dv]
    if layout == "bhtd":
        out = [x.transpose(1, 2) for x in out]
    return [x.float().cpu() for x in out], taken


def _oracle(q, k, v, pos, o, lse, do, scale=None, layout="bthd"):
    if layout == "bhtd":
        o = o.transpose(1, 2)
    return oatt.sparse_attention_bwd(q, k, v, pos, o.cpu().to(q.dtype), lse.cpu(), do, None, scale)


@pytest.mark.parametrize(
    "batch,tq,tk,heads,topk,dtype,layout,scale,invalid",
    [
        (1, 128, 128, 2, 64, torch.float16, "bthd", None, 0.0),   # geoweave/kernels.py:27-41 shape
        (2, 300, 300, 4, 77, torch.bfloat16, "bthd", 0.1, 0.3),   # ragged -1 tails
        (1, 1000, 700, 3, 100, torch.bfloat16, "bhtd", None, 0.0),  # T != S, bhtd
        (2, 513, 1029, 16, 64, torch.float16, "bthd", 0.2, 0.1),  # T, S off every tile size
        (1, 33, 5000, 1, 512, torch.bfloat16, "bthd", None, 0.0),  # one head, long key range
        (1, 64, 41000, 2, 512, torch.bfloat16, "bthd", None, 0.0),  # selection words in 3 key chunks
    ],
)
def test_dense_backward_matches_oracle(gpu_device, batch, tq, tk, heads, topk, dtype, layout, scale, invalid):
    q = workloads.attention_inputs(1, batch, dtype, tokens=tq, heads=heads, seed=tq)[0]
    _, k, v = workloads.attention_inputs(1, batch, dtype, tokens=tk, heads=heads, seed=tk + 1)
    pos = workloads.random_positions(batch, tq, tk, topk, seed=tq + tk, invalid_fraction=invalid)
    if invalid > 0:
        pos[:, ::7, -3:] = tk  # out-of-range entries are masked like -1
    do = torch.randn(batch, tq, heads, 64, generator=torch.Generator().manual_seed(3)).to(dtype)
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos, scale, layout)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc, layout)
    assert taken == "dense"
    rq, rk, rv = _oracle(q, k, v, pos, o, lse, do, scale, layout)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)


def test_dense_backward_empty_rows_and_unselected_keys(gpu_device):
    T, S, H, K = 700, 900, 4, 40
    q = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=T, heads=H, seed=5)[0]
    _, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=S, heads=H, seed=6)
    pos = workloads.random_positions(1, T, S, K, seed=7)
    pos[0, 10:50] = -1  # rows with nothing valid: lse = -inf, dq = 0
    pos[0, 60, 5:] = S + 3
    pos = torch.where(pos >= 800, torch.full_like(pos, -1), pos)  # keys 800.. never selected
    do = torch.randn(1, T, H, 64, generator=torch.Generator().manual_seed(8)).bfloat16()
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert taken == "dense"
    assert torch.all(dq[0, 10:50] == 0)
    assert torch.all(dk[0, 800:] == 0) and torch.all(dv[0, 800:] == 0)
    rq, rk, rv = _oracle(q, k, v, pos, o, lse, do)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)


def test_repeated_positions_take_the_csr_path(gpu_device):
    T, H, K = 400, 4, 64
    q, k, v = workloads.attention_inputs(1, 2, torch.bfloat16, tokens=T, heads=H, seed=11)
    pos = workloads.random_positions(2, T, T, K, seed=12)
    pos[1, 77, 9] = pos[1, 77, 3]  # one repeat in batch element 1: it counts twice
    do = torch.randn(2, T, H, 64, generator=torch.Generator().manual_seed(13)).bfloat16()
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert taken == "csr"
    rq, rk, rv = _oracle(q, k, v, pos, o, lse, do)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)


@pytest.mark.parametrize("where", ["k", "v", "q", "do"])
def test_nonfinite_inputs_take_the_csr_path(gpu_device, where):
    # inf / nan in rows no query selects (k, v) or in a query row (q, dO): the reference reads
    # only selected rows, so every gradient the oracle leaves finite must stay finite and equal.
    T, S, H, K = 300, 400, 2, 32
    q = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=T, heads=H, seed=21)[0]
    _, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=S, heads=H, seed=22)
    pos = workloads.random_positions(1, T, 390, K, seed=23)  # keys 390.. never selected
    do = torch.randn(1, T, H, 64, generator=torch.Generator().manual_seed(24)).bfloat16()
    if where == "k":
        k[0, 395, 1, 7] = float("inf")
    elif where == "v":
        v[0, 392, 0, 3] = float("nan")
    elif where == "q":
        q[0, 17, 1, 0] = float("inf")
    else:
        do[0, 250, 0, 9] = float("nan")
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert taken == "csr"
    rq, rk, rv = _oracle(q, k, v, pos, o, lse, do)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        fin = torch.isfinite(ref)
        assert torch.equal(torch.isfinite(got), fin)
        torch.testing.assert_close(got[fin], ref[fin], **TOL)


def test_dense_backward_is_bitwise_reproducible(gpu_device):
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=3000, seed=31)
    pos = workloads.distinct_positions(1, 3000, 3000, 256, seed=32, hub=7)
    do = torch.randn(1, 3000, 16, 64, generator=torch.Generator().manual_seed(33)).bfloat16()
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    a, ta = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    b, tb = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert ta == tb == "dense"
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_fp16_small_gradients_keep_their_precision(gpu_device):
    # dO of order 1e-5: ds = p (dp - delta) is far below fp16's normal range unless scaled;
    # the relative error must stay at the level of the unscaled case.
    T, H, K = 600, 4, 128
    q, k, v = workloads.attention_inputs(1, 1, torch.float16, tokens=T, heads=H, seed=41)
    pos = workloads.random_positions(1, T, T, K, seed=42)
    do = (torch.randn(1, T, H, 64, generator=torch.Generator().manual_seed(43)) * 1e-5).half()
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert taken == "dense"
    rq, rk, rv = _oracle(q, k, v, pos, o, lse, do)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        m = ref.abs().max()
        torch.testing.assert_close(got / m, ref / m, **TOL)


def test_dense_equals_csr_at_c1(gpu_device):
    # Config C1's attention shape (S=4 views, N=5496, H=16, K=1024) with distinct positions:
    # the dense passes against the oracle on every row, and against the CSR backward.
    views, K = 4, 1024
    q, k, v = workloads.attention_inputs(views, 1, torch.bfloat16)
    n = q.shape[1]
    pos = workloads.distinct_positions(1, n, n, K, seed=views, hub=100)
    do = torch.randn(1, n, 16, 64, generator=torch.Generator().manual_seed(views)).bfloat16()
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert taken == "dense"
    (cq, ck, cv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc, path="csr")
    assert taken == "csr"
    for x, y in ((dq, cq), (dk, ck), (dv, cv)):
        torch.testing.assert_close(x, y, **TOL)
    rq, rk, rv = _oracle(q, k, v, pos, o, lse, do)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dv, rv, **TOL)


def test_dense_backward_training_shape(gpu_device):
    # Config C4 (B=2, S=24 views, N=32976, H=16, D=64, K=1024) with distinct positions and a
    # key every query lists: the dense passes against the CSR backward on every element,
    # against the oracle on sampled query rows and keys, and the exact invariants
    # sum_s dV = sum_t dO and sum_s dK = 0 per head.
    views, B, K = 24, 2, 1024
    q, k, v = workloads.attention_inputs(views, B, torch.bfloat16)
    n = q.shape[1]
    g = torch.Generator().manual_seed(views)
    pos = workloads.distinct_positions(B, n, n, K, seed=views, hub=12345)
    do = torch.randn(B, n, 16, 64, generator=g).bfloat16()
    qd, kd, vd, pd, o, lse, sc = _fwd(q, k, v, pos)
    (dq, dk, dv), taken = _bwd(do, qd, kd, vd, pd, o, lse, sc)
    assert taken == "dense"
    (cq, ck, cv), _ = _bwd(do, qd, kd, vd, pd, o, lse, sc, path="csr")
    for x, y in ((dq, cq), (dk, ck), (dv, cv)):
        torch.testing.assert_close(x, y, **TOL)
    del cq, ck, cv
    o, lse = o.cpu(), lse.cpu()
    rows = torch.randperm(n, generator=g)[:96]
    rq, _, _ = oatt.sparse_attention_bwd(q[:, rows], k, v, pos[:, rows], o[:, rows], lse[:, rows], do[:, rows])
    torch.testing.assert_close(dq[:, rows], rq, **TOL)
    keys = torch.cat([torch.tensor([12345]), torch.randperm(n, generator=g)[:15]])
    rk, rv = oatt.sparse_attention_bwd_keys(q, k, v, pos, o, lse, do, keys)
    torch.testing.assert_close(dk[:, keys], rk, **TOL)
    torch.testing.assert_close(dv[:, keys], rv, **TOL)
    torch.testing.assert_close(dv.sum(1), do.float().sum(1), atol=0.5, rtol=1e-2)
    assert dk.sum(1).abs().max() < 0.5


def test_autograd_with_detached_attention_mass(gpu_device):
    # The reference presets' training: o feeds the loss, attn_sum only a detached indexer
    # loss, so attn_sum brings no gradient and the dense passes run.
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=512, seed=51)
    pos = workloads.random_positions(1, 512, 512, 128, seed=52)
    do = torch.randn(1, 512, 16, 64, generator=torch.Generator().manual_seed(53)).bfloat16()
    qd, kd, vd = (x.cuda().requires_grad_() for x in (q, k, v))
    o, attn = sifa.sparse_index_flash_attn_func(qd, kd, vd, pos.cuda())
    p = attn.detach()
    (o.float() * do.cuda().float()).sum().backward()
    assert _backward.last_path == "dense"
    assert torch.isfinite(p).all()
    o_ref, _, lse_ref = oatt.sparse_attention(q, k, v, pos)
    rq, rk, rv = oatt.sparse_attention_bwd(q, k, v, pos, o_ref.to(q.dtype), lse_ref, do)
    torch.testing.assert_close(qd.grad.float().cpu(), rq, **TOL)
    torch.testing.assert_close(kd.grad.float().cpu(), rk, **TOL)
    torch.testing.assert_close(vd.grad.float().cpu(), rv, **TOL)
