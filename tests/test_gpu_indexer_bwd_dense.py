"""GPU checks of the indexer backward's masked dense passes (gw_indexer_topk_bwd_dense):
against the oracle (oracle/indexer.py, which restates the reference's
_indexer_topk_bwd_kernel, sparse_topk_indexer.py:1847-1944), against the CSR path, on
ragged shapes, invalid positions, every head count, row groups cut between persistent
workgroups, repeated positions and non-finite inputs (both reported back and redone by the
CSR path), and for bitwise reproducibility.
"""
import pytest
import torch

from geoweave_amd import _lib, workloads
from geoweave_amd.custom_indexer import _backward as ib
from oracle import indexer as oidx

pytestmark = pytest.mark.gpu
TOL = dict(atol=2e-2, rtol=2e-2)


def _dyadic(shape, g, vals=(-1.0, -0.5, 0.0, 0.5, 1.0)):
    t = torch.tensor(vals)
    return t[torch.randint(0, len(vals), shape, generator=g)]


def _run(path, q, k, w, idx, grad, scale=0.125):
    old = ib.BACKWARD_PATH
    ib.BACKWARD_PATH = path
    try:
        dq, dk, dw = ib.indexer_topk_backward(q.cuda(), k.cuda(), w.cuda(), idx.cuda(), grad.cuda(), scale)
        torch.cuda.synchronize()
    finally:
        ib.BACKWARD_PATH = old
    return dq.float().cpu(), dk.float().cpu(), dw.float().cpu(), ib.last_path


def _oracle(q, k, w, idx, grad, scale=0.125):
    # Invalid positions contribute nothing: point them at key 0 with a zero gradient.
    bad = (idx < 0) | (idx >= k.shape[1])
    return oidx.indexer_topk_bwd(q, k, w, torch.where(bad, 0, idx), torch.where(bad, 0, grad.float()), scale)


@pytest.mark.parametrize("heads", [1, 2, 4, 8])
def test_dense_matches_oracle_exactly_on_dyadic_inputs(gpu_device, heads):
    # Dyadic q, k, w and gradients: every z, every w k and every fp32 sum is exact, so the
    # dense passes equal the oracle bit for bit. Ragged T and S (not multiples of 32 or of
    # the 256-row groups), K not a multiple of 4, a key chosen by every query.
    g = torch.Generator().manual_seed(100 + heads)
    B, T, S, K = 2, 613, 1001, 93
    print(f"[idx dense] dyadic heads={heads} T={T} S={S} K={K}", flush=True)
    q = _dyadic((B, T, heads, 64), g).bfloat16()
    k = _dyadic((B, S, heads, 64), g).bfloat16()
    w = _dyadic((B, S, heads), g, (-0.5, 0.75, 1.0, 1.25, 1.5)).bfloat16()
    idx = workloads.random_positions(B, T, S, K, seed=heads)
    idx[0, :, 0] = torch.where((idx[0] == 7).any(-1), idx[0, :, 0], 7)  # key 7 in every row of b = 0
    grad = (torch.randint(-8, 9, (B, T, K), generator=g).float() / 8).bfloat16()
    dq, dk, dw, path = _run("dense", q, k, w, idx, grad)
    assert path == "dense"
    rq, rk, rw = _oracle(q, k, w, idx, grad)
    assert torch.equal(dq, rq.bfloat16().float())
    assert torch.equal(dk, rk.bfloat16().float())
    assert torch.equal(dw, rw.bfloat16().float())


def test_dense_matches_csr_and_oracle_with_invalid_positions(gpu_device):
    # Random bf16 inputs with ragged -1 tails and positions past S: dense against the oracle
    # (0.1 % relu-gate flips allowed) and against the CSR path.
    g = torch.Generator().manual_seed(7)
    B, T, S, K = 2, 1500, 2600, 200
    q = torch.randn(B, T, 4, 64, generator=g).bfloat16()
    k = torch.randn(B, S, 4, 64, generator=g).bfloat16()
    w = torch.randn(B, S, 4, generator=g).bfloat16()
    idx = workloads.random_positions(B, T, S, K, seed=8, invalid_fraction=0.4)
    idx[1, ::7, -1] = S + 5  # past the end: skipped like -1
    grad = torch.randn(B, T, K, generator=g).bfloat16()
    dq, dk, dw, path = _run("dense", q, k, w, idx, grad)
    assert path == "dense"
    cq, ck, cw, cpath = _run("csr", q, k, w, idx, grad)
    assert cpath == "csr"
    rq, rk, rw = _oracle(q, k, w, idx, grad)
    for got, csr, ref in ((dq, cq, rq), (dk, ck, rk), (dw, cw, rw)):
        bad = ~torch.isclose(got, ref, **TOL)
        assert bad.float().mean() <= 1e-3, f"{int(bad.sum())} of {bad.numel()} outside tolerance"
        bad = ~torch.isclose(got, csr, **TOL)
        assert bad.float().mean() <= 1e-3, f"dense vs csr: {int(bad.sum())} of {bad.numel()}"


@pytest.mark.parametrize("B,T,S,K", [(1, 40, 70, 16), (2, 4100, 4100, 256), (1, 257, 33, 33)])
def test_stream_k_splits_and_tiny_shapes(gpu_device, B, T, S, K):
    # (1, 40, 70): fewer iterations than workgroups; (2, 4100, 4100): every row group is cut
    # between several persistent workgroups (partials summed by the fixup pass); (1, 257, 33):
    # one key block past a full row group. Dyadic inputs: exact against the oracle.
    g = torch.Generator().manual_seed(T + S)
    print(f"[idx dense] stream-K B={B} T={T} S={S} K={K}", flush=True)
    q = _dyadic((B, T, 4, 64), g).bfloat16()
    k = _dyadic((B, S, 4, 64), g).bfloat16()
    w = _dyadic((B, S, 4), g, (-0.5, 0.75, 1.0, 1.25)).bfloat16()
    idx = workloads.random_positions(B, T, S, K, seed=3)
    grad = (torch.randint(-4, 5, (B, T, K), generator=g).float() / 4).bfloat16()
    dq, dk, dw, path = _run("dense", q, k, w, idx, grad)
    assert path == "dense"
    rq, rk, rw = _oracle(q, k, w, idx, grad)
    assert torch.equal(dq, rq.bfloat16().float())
    assert torch.equal(dk, rk.bfloat16().float())
    assert torch.equal(dw, rw.bfloat16().float())


def test_repeated_position_and_nonfinite_key_take_the_csr_path(gpu_device):
    # A position listed twice in a row counts twice (the reference adds both entries); a
    # non-finite key that no query selected must not reach any gradient. The dense passes
    # flag both cases and the call is redone by the CSR path, which matches the oracle.
    g = torch.Generator().manual_seed(11)
    B, T, S, K = 2, 300, 500, 40
    q = _dyadic((B, T, 2, 64), g).bfloat16()
    k = _dyadic((B, S, 2, 64), g).bfloat16()
    w = _dyadic((B, S, 2), g, (0.5, 1.0, 1.5)).bfloat16()
    idx = workloads.random_positions(B, T, S, K, seed=12)
    grad = torch.randn(B, T, K, generator=g).bfloat16()
    dup = idx.clone()
    dup[1, 17, 3] = dup[1, 17, 9]
    dq, dk, dw, path = _run("dense", q, k, w, dup, grad)
    assert path == "csr"
    rq, rk, rw = _oracle(q, k, w, dup, grad)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dw, rw, **TOL)
    idx[0][idx[0] == 13] = -1  # no query of batch element 0 selects key 13
    kinf = k.clone()
    kinf[0, 13, 1, 5] = float("inf")
    dq, dk, dw, path = _run("dense", q, kinf, w, idx, grad)
    assert path == "csr"
    rq, rk, rw = _oracle(q, k, w, idx, grad)
    torch.testing.assert_close(dq, rq, **TOL)
    torch.testing.assert_close(dk, rk, **TOL)
    torch.testing.assert_close(dw, rw, **TOL)


def test_dense_is_bitwise_reproducible_and_reports_route_flags(gpu_device):
    g = torch.Generator().manual_seed(21)
    B, T, S, K = 2, 2000, 2100, 128
    q = torch.randn(B, T, 4, 64, generator=g).bfloat16().cuda()
    k = torch.randn(B, S, 4, 64, generator=g).bfloat16().cuda()
    w = torch.randn(B, S, 4, generator=g).bfloat16().cuda()
    idx = workloads.random_positions(B, T, S, K, seed=22).cuda()
    idx[1, 5, 1] = idx[1, 5, 0]  # batch element 1 only
    grad = torch.randn(B, T, K, generator=g).bfloat16().cuda()
    lib = _lib.load()
    outs = []
    for _ in range(2):
        dq, dk, dw = torch.full_like(q, 7.0), torch.full_like(k, 7.0), torch.full_like(w, 7.0)
        route = torch.full((B,), 5, dtype=torch.int32, device="cuda")
        nbytes = int(lib.gw_indexer_topk_bwd_dense_workspace_size(B, T, S, 4, 64, K))
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        rc = lib.gw_indexer_topk_bwd_dense(
            _lib.GW_DTYPE_BF16, q.data_ptr(), k.data_ptr(), w.data_ptr(), idx.data_ptr(), grad.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dw.data_ptr(), B, T, S, 4, 64, K, 0.125, route.data_ptr(),
            ws.data_ptr(), nbytes, _lib.stream_handle(q.device))
        _lib.check(rc, "gw_indexer_topk_bwd_dense")
        torch.cuda.synchronize()
        assert route.tolist() == [0, 1]
        # the flagged element is left untouched
        assert bool((dq[1] == 7.0).all()) and bool((dk[1] == 7.0).all()) and bool((dw[1] == 7.0).all())
        outs.append((dq[0].cpu(), dk[0].cpu(), dw[0].cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    rq, rk, rw = _oracle(q[:1].cpu(), k[:1].cpu(), w[:1].cpu(), idx[:1].cpu(), grad[:1].cpu())
    for got, ref in ((outs[0][0], rq[0]), (outs[0][1], rk[0]), (outs[0][2], rw[0])):
        bad = ~torch.isclose(got.float(), ref, **TOL)
        assert bad.float().mean() <= 1e-3, f"{int(bad.sum())} of {bad.numel()} outside tolerance"


def test_unsupported_inputs_are_refused(gpu_device):
    lib = _lib.load()
    x = torch.empty(64, dtype=torch.uint8, device="cuda")
    route = torch.empty(1, dtype=torch.int32, device="cuda")
    p = x.data_ptr()
    args = (p, p, p, p, p, p, p, p)
    for code, S, K in ((_lib.GW_DTYPE_FP16, 100, 8), (_lib.GW_DTYPE_BF16, 65537, 8), (_lib.GW_DTYPE_BF16, 100, 2049)):
        rc = lib.gw_indexer_topk_bwd_dense(code, *args, 1, 4, S, 4, 64, K, 0.125, route.data_ptr(), p, 64,
                                           _lib.stream_handle(x.device))
        assert rc == 2, lib.gw_last_error()
