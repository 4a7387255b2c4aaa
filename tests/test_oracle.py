"""Pins the CPU oracle (oracle/) against fixtures, brute force, closed forms and invariants.

CPU only. Each check is chosen so that a plausible slip in the oracle (a dropped term, a
wrong sign, a transposed operand, a head/key index mix-up) fails at least one of them.
"""
import json
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import indexer as oidx
from oracle.topk_check import check_topk_rows

GOLDEN = Path(__file__).resolve().parent / "golden"


def _t(x, dtype=torch.float32):
    return torch.tensor(x, dtype=dtype)


# ----------------------------------------------------------------------------- indexer


@pytest.mark.parametrize("case", json.loads((GOLDEN / "indexer_kat.json").read_text()), ids=lambda c: c["name"])
def test_indexer_scores_and_topk_match_golden(case):
    q = _t(case["q"]).unsqueeze(0)
    k = _t(case["k"]).unsqueeze(0)
    w = _t(case["w"]).unsqueeze(0)
    mask = None if case["mask"] is None else _t(case["mask"]).unsqueeze(0)
    sc = oidx.indexer_scores(q, k, w, mask, case["scale"])
    torch.testing.assert_close(sc[0], _t(case["scores"]), atol=1e-6, rtol=1e-6)
    idx, val = oidx.indexer_topk(q, k, w, mask, case["topk"], case["scale"])
    got = sorted(idx[0].sort(-1).values.tolist())
    assert [sorted(r) for r in idx[0].tolist()] == case["expected_sets"], got
    torch.testing.assert_close(val, sc.gather(-1, idx.long()))


def _view_bias_case(case):
    q = _t(case["q"]).unsqueeze(0)
    k = _t(case["k"]).unsqueeze(0)
    w = _t(case["w"]).unsqueeze(0)
    mask = None if case["mask"] is None else _t(case["mask"]).unsqueeze(0)
    vb = (torch.tensor(case["q_view_ids"]), torch.tensor(case["s_view_ids"]), _t(case["view_bias"]))
    return q, k, w, mask, vb


@pytest.mark.parametrize("case", json.loads((GOLDEN / "indexer_view_bias_kat.json").read_text()),
                         ids=lambda c: c["name"])
def test_indexer_view_bias_matches_golden(case):
    # fp64 loops of the reference's view-bias cases (tests/indexer_projected_tests.py:64-243)
    q, k, w, mask, vb = _view_bias_case(case)
    sc = oidx.indexer_scores(q, k, w, mask, case["scale"], view_bias=vb)
    torch.testing.assert_close(sc[0], _t(case["scores"]), atol=1e-6, rtol=1e-6)
    idx, val = oidx.indexer_topk(q, k, w, mask, case["topk"], case["scale"], view_bias=vb)
    rep = check_topk_rows(_t(case["scores"]), idx[0], case["topk"])
    assert rep.ok, rep
    if "table_grad_of_sum" in case:
        g = oidx.view_bias_grad(idx, torch.ones(idx.shape), vb[0], vb[1], vb[2].shape)
        torch.testing.assert_close(g, _t(case["table_grad_of_sum"]), atol=0, rtol=0)


def test_view_bias_grad_equals_autograd_of_the_gathered_term():
    # the scatter restatement against autograd of table[b, q_view, s_view[idx]] (an
    # independent route: index-gather backward)
    g = torch.Generator().manual_seed(5)
    B, T, S, K, Vq, Vs = 2, 13, 17, 5, 3, 4
    qv = torch.randint(0, Vq, (B, T), generator=g)
    sv = torch.randint(0, Vs, (B, S), generator=g)
    idx = torch.stack([torch.stack([torch.randperm(S, generator=g)[:K] for _ in range(T)]) for _ in range(B)])
    table = torch.randn(B, Vq, Vs, generator=g, requires_grad=True)
    gs = torch.randn(B, T, K, generator=g)
    term = oidx.view_bias_term(qv, sv, table)  # [B, T, S]
    (term.gather(-1, idx) * gs).sum().backward()
    torch.testing.assert_close(oidx.view_bias_grad(idx, gs, qv, sv, table.shape), table.grad)
    # a transposed lookup (s view as row) would fail this: Vq != Vs and ids differ
    assert oidx.view_bias_term(qv, sv, table.detach())[0, 0, 0] == table[0, qv[0, 0], sv[0, 0]]


def test_indexer_scores_closed_form_single_head_unit_gate():
    # Hi = 1, w = 1  =>  score = relu(scale * q k^T)
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 9, 1, 16, generator=g)
    k = torch.randn(2, 11, 1, 16, generator=g)
    w = torch.ones(2, 11, 1)
    sc = oidx.indexer_scores(q, k, w, None, 0.25)
    ref = torch.relu(0.25 * torch.einsum("btd,bsd->bts", q[:, :, 0], k[:, :, 0]))
    torch.testing.assert_close(sc, ref, atol=1e-6, rtol=1e-6)


def test_indexer_scores_orthogonal_query_is_zero_and_heads_use_key_gate():
    q = torch.zeros(1, 1, 2, 4)
    q[0, 0, 0, 0] = 1.0  # head 0 looks at dim 0; head 1 is zero
    k = torch.zeros(1, 3, 2, 4)
    k[0, 0, 0, 1] = 5.0  # orthogonal to q -> 0
    k[0, 1, 0, 0] = 2.0  # z = 2 on head 0
    k[0, 2, 1, 0] = 7.0  # only head 1, where q is 0 -> 0
    w = torch.tensor([[[3.0, 100.0], [-1.5, 100.0], [9.0, 100.0]]])
    sc = oidx.indexer_scores(q, k, w, None, 1.0)
    # key 1: w[1, head0] * relu(2) = -3 (the gate is indexed by the KEY token)
    torch.testing.assert_close(sc[0, 0], torch.tensor([0.0, -3.0, 0.0]))


def test_indexer_scores_brute_force_random():
    g = torch.Generator().manual_seed(1)
    B, T, S, H, D = 2, 5, 13, 3, 6
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, S, H, D, generator=g)
    w = torch.randn(B, S, H, generator=g)
    mask = torch.randn(B, T, S, generator=g)
    sc = oidx.indexer_scores(q, k, w, mask, 0.3, key_chunk=4, query_chunk=2)
    ref = torch.zeros(B, T, S, dtype=torch.float64)
    for b in range(B):
        for t in range(T):
            for s in range(S):
                acc = 0.0
                for h in range(H):
                    z = sum(float(q[b, t, h, d]) * float(k[b, s, h, d]) for d in range(D))
                    acc += float(w[b, s, h]) * max(0.3 * z, 0.0)
                ref[b, t, s] = acc + float(mask[b, t, s])
    torch.testing.assert_close(sc.double(), ref, atol=1e-5, rtol=1e-5)


def test_indexer_topk_matches_full_sort():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 40, 4, 8, generator=g)
    k = torch.randn(1, 300, 4, 8, generator=g)
    w = 1 + 0.2 * torch.randn(1, 300, 4, generator=g)
    idx, val = oidx.indexer_topk(q, k, w, None, 37, 0.125, query_chunk=7)
    sc = oidx.indexer_scores(q, k, w, None, 0.125)
    order = sc.argsort(dim=-1, descending=True)[..., :37]
    assert torch.equal(idx.long().sort(-1).values, order.sort(-1).values)
    torch.testing.assert_close(val, sc.gather(-1, idx.long()))
    sel = oidx.selected_scores(q, k, w, idx, 0.125)
    torch.testing.assert_close(sel, val, atol=1e-5, rtol=1e-5)


def test_indexer_topk_caps_k_at_source_length():
    q = torch.randn(1, 3, 1, 4)
    k = torch.randn(1, 5, 1, 4)
    w = torch.ones(1, 5, 1)
    idx, _ = oidx.indexer_topk(q, k, w, None, 1024, 0.5)
    assert idx.shape == (1, 3, 5)
    assert all(sorted(r) == list(range(5)) for r in idx[0].tolist())


def test_indexer_bwd_matches_autograd_of_torch_path():
    # The reference's torch backend differentiates scores.gather(-1, topk_indices)
    # (indexer.py:600-603); the explicit kernel formula must agree with it.
    g = torch.Generator().manual_seed(3)
    B, T, S, H, D, K = 2, 6, 20, 4, 8, 5
    q = torch.randn(B, T, H, D, generator=g, requires_grad=True)
    k = torch.randn(B, S, H, D, generator=g, requires_grad=True)
    w = torch.randn(B, S, H, generator=g, requires_grad=True)
    sc = oidx.indexer_scores(q, k, w, None, 0.125)
    idx = sc.detach().topk(K, dim=-1).indices
    gsc = torch.randn(B, T, K, generator=g)
    sc.gather(-1, idx).backward(gsc)
    dq, dk, dw = oidx.indexer_topk_bwd(q.detach(), k.detach(), w.detach(), idx.int(), gsc, 0.125)
    torch.testing.assert_close(dq, q.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(dk, k.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(dw, w.grad, atol=1e-5, rtol=1e-5)


# ----------------------------------------------------------------------------- attention


def _fixture():
    f = json.loads((GOLDEN / "attn_fixture.json").read_text())
    q = _t(f["q"]).unsqueeze(0)
    k = _t(f["k"]).unsqueeze(0)
    v = _t(f["v"]).unsqueeze(0)
    do = _t(f["do"]).unsqueeze(0)
    pos = torch.tensor(f["kv_positions"], dtype=torch.int32).unsqueeze(0)
    dattn = _t(f["dattn"]).unsqueeze(0)
    return f, q, k, v, do, pos, dattn


def test_sparse_attention_matches_golden_bruteforce():
    f, q, k, v, do, pos, dattn = _fixture()
    o, asum, lse = oatt.sparse_attention(q, k, v, pos, f["scale"], query_chunk=2)
    torch.testing.assert_close(o[0], _t(f["o"]), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(asum[0], _t(f["attn_sum"]), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(lse[0], _t(f["lse"]), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("with_dattn", [False, True])
def test_sparse_attention_bwd_matches_golden_and_autograd(with_dattn):
    f, q, k, v, do, pos, dattn = _fixture()
    da = dattn if with_dattn else None
    o, asum, lse = oatt.sparse_attention(q, k, v, pos, f["scale"])
    dq, dk, dv = oatt.sparse_attention_bwd(q, k, v, pos, o, lse, do, da, f["scale"], query_chunk=2)
    aq, ak, av = oatt.sparse_attention_autograd(q, k, v, pos, do, da, f["scale"])
    torch.testing.assert_close(dq, aq, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(dk, ak, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(dv, av, atol=1e-5, rtol=1e-5)
    if with_dattn:
        torch.testing.assert_close(dq[0], _t(f["dq"]), atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(dk[0], _t(f["dk"]), atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(dv[0], _t(f["dv"]), atol=1e-5, rtol=1e-5)


def test_sparse_attention_dense_positions_equal_sdpa():
    g = torch.Generator().manual_seed(4)
    B, T, H, D = 2, 17, 3, 8
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, T, H, D, generator=g)
    v = torch.randn(B, T, H, D, generator=g)
    pos = torch.arange(T, dtype=torch.int32).view(1, 1, T).expand(B, T, T).contiguous()
    o, asum, lse = oatt.sparse_attention(q, k, v, pos, None, query_chunk=5)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
    torch.testing.assert_close(o, ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(asum.sum(-1), torch.full((B, T), float(H)), atol=1e-5, rtol=1e-5)
    s = torch.einsum("bthd,bshd->bhts", q, k) / math.sqrt(D)
    torch.testing.assert_close(lse, torch.logsumexp(s, -1).transpose(1, 2), atol=1e-5, rtol=1e-5)


def test_sparse_attention_row_permutation_invariance():
    g = torch.Generator().manual_seed(5)
    B, T, S, H, D, K = 1, 6, 30, 2, 8, 9
    q, k, v = (torch.randn(B, n, H, D, generator=g) for n in (T, S, S))
    pos = torch.stack([torch.randperm(S, generator=g)[:K] for _ in range(T)]).int().unsqueeze(0)
    perm = torch.randperm(K, generator=g)
    o1, a1, _ = oatt.sparse_attention(q, k, v, pos)
    o2, a2, _ = oatt.sparse_attention(q, k, v, pos[..., perm].contiguous())
    torch.testing.assert_close(o1, o2, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(a1[..., perm], a2, atol=1e-6, rtol=1e-6)


def test_sparse_attention_invalid_rows_and_bwd_invariants():
    g = torch.Generator().manual_seed(6)
    B, T, S, H, D, K = 1, 8, 25, 2, 4, 6
    q, k, v = (torch.randn(B, n, H, D, generator=g) for n in (T, S, S))
    pos = torch.stack([torch.randperm(S, generator=g)[:K] for _ in range(T)]).int().unsqueeze(0)
    bad = pos.clone()
    bad[0, 1, 3:] = -1
    bad[0, 2, :] = -1  # no valid candidate at all
    bad[0, 3, 0] = S   # past the end is masked too
    o, asum, lse = oatt.sparse_attention(q, k, v, bad)
    assert torch.all(o[0, 2] == 0) and torch.all(asum[0, 2] == 0) and torch.isinf(lse[0, 2]).all()
    assert asum[0, 1, 3:].abs().max() == 0 and asum[0, 3, 0] == 0
    do = torch.randn(B, T, H, D, generator=g)
    # Exact invariants for all-valid rows and no dattn: sum_s dK = 0, sum_s dV = sum_t dO.
    o, asum, lse = oatt.sparse_attention(q, k, v, pos)
    dq, dk, dv = oatt.sparse_attention_bwd(q, k, v, pos, o, lse, do)
    torch.testing.assert_close(dk.sum(1), torch.zeros(B, H, D), atol=1e-5, rtol=0)
    torch.testing.assert_close(dv.sum(1), do.sum(1), atol=1e-5, rtol=1e-5)


# ----------------------------------------------------------------------------- top-k checker


def test_topk_checker_accepts_ties_and_rejects_planted_mistakes():
    g = torch.Generator().manual_seed(7)
    rows, S, K = 4, 50, 10
    sc = torch.randn(rows, S, generator=g)
    # plant an exact tie at the k-th place of row 0
    srt = sc[0].sort(descending=True)
    sc[0, srt.indices[K]] = srt.values[K - 1]
    ref = sc.topk(K, dim=-1).indices
    assert check_topk_rows(sc, ref, K).ok
    swapped = ref.clone()
    pos_kth = (ref[0] == srt.indices[K - 1]).nonzero()
    if pos_kth.numel():
        swapped[0, pos_kth[0, 0]] = srt.indices[K]
        rep = check_topk_rows(sc, swapped, K)
        assert rep.ok and rep.rows_tie_swapped >= 1
    wrong = ref.clone()
    wrong[1, 0] = sc[1].argmin()
    assert not check_topk_rows(sc, wrong, K).ok
    dup = ref.clone()
    dup[2, 1] = dup[2, 0]
    assert not check_topk_rows(sc, dup, K).ok
    oob = ref.clone()
    oob[3, 0] = -1
    assert not check_topk_rows(sc, oob, K).ok


def test_key_subset_backward_helpers_match_full_backward():
    # The key-subset helpers (used for full-size GPU checks) must equal the full oracle
    # backward on the rows they return.
    g = torch.Generator().manual_seed(8)
    B, T, S, H, D, K = 2, 40, 30, 3, 8, 7
    q, do = (torch.randn(B, T, H, D, generator=g) for _ in range(2))
    k, v = (torch.randn(B, S, H, D, generator=g) for _ in range(2))
    pos = torch.stack([torch.stack([torch.randperm(S, generator=g)[:K] for _ in range(T)]) for _ in range(B)]).int()
    pos[0, 3, 2] = pos[0, 3, 1]  # a duplicate entry
    o, _, lse = oatt.sparse_attention(q, k, v, pos)
    dq, dk, dv = oatt.sparse_attention_bwd(q, k, v, pos, o, lse, do)
    keys = torch.tensor([0, 7, pos[0, 3, 1].item(), 29])
    sk, sv = oatt.sparse_attention_bwd_keys(q, k, v, pos, o, lse, do, keys)
    torch.testing.assert_close(sk, dk[:, keys], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(sv, dv[:, keys], atol=1e-5, rtol=1e-5)
    w = torch.randn(B, S, H, generator=g)
    gs = torch.randn(B, T, K, generator=g)
    _, ik, iw = oidx.indexer_topk_bwd(q, k, w, pos, gs, 0.3)
    hk, hw = oidx.indexer_topk_bwd_keys(q, k, w, pos, gs, keys, 0.3)
    torch.testing.assert_close(hk, ik[:, keys], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(hw, iw[:, keys], atol=1e-5, rtol=1e-5)


def test_kl_oracle_forward_equals_scipy_entropy_and_brute_force():
    # eps = 0 reduces the row loss to the textbook KL(p || softmax(z)) = scipy.stats.entropy.
    from scipy.stats import entropy
    from oracle import kl_loss as okl

    g = torch.Generator().manual_seed(11)
    a = torch.rand(2, 3, 17, generator=g, dtype=torch.float64) + 1e-3
    z = torch.randn(2, 3, 17, generator=g, dtype=torch.float64) * 3
    rows = okl.kl_row_losses(a, z, eps=0.0)
    for r, (ar, zr) in enumerate(zip(a.reshape(-1, 17), z.reshape(-1, 17))):
        q = torch.softmax(zr, -1)
        assert abs(float(rows[r]) - entropy(ar.numpy(), q.numpy())) < 1e-12
    # eps > 0: a pure-Python loop over the reference's per-element formula
    # (indexer_kl_fused.py:76-91) with log-sum-exp written out.
    eps = 1e-2
    ar = [float(x) for x in a[1, 2]]
    zr = [float(x) for x in z[1, 2]]
    tot = sum(ar)
    lse = math.log(sum(math.exp(x) for x in zr))
    want = sum((x / (tot + eps)) * (math.log(x / (tot + eps) + eps) - (y - lse)) for x, y in zip(ar, zr))
    assert abs(float(okl.kl_row_losses(a, z, eps)[5]) - want) < 1e-12
    assert abs(float(okl.kl_loss(a, z, eps)) - float(okl.kl_row_losses(a, z, eps).mean())) < 1e-15


def test_kl_oracle_invariants():
    from oracle import kl_loss as okl

    g = torch.Generator().manual_seed(12)
    z = torch.randn(1, 4, 32, generator=g, dtype=torch.float64)
    # p == softmax(z) and eps -> 0: the loss vanishes and so does d_logits.
    p = torch.softmax(z, -1)
    assert float(okl.kl_loss(p, z, eps=0.0).abs()) < 1e-14
    _, dz = okl.kl_loss_bwd(p, z, 1.0, eps=0.0)
    assert float(dz.abs().max()) < 1e-14
    # a shift of the logits per row changes nothing; with eps = 0 neither does a scale of attn.
    a = torch.rand(1, 4, 32, generator=g, dtype=torch.float64)
    base = okl.kl_row_losses(a, z, 0.0)
    assert torch.allclose(okl.kl_row_losses(a, z + torch.randn(1, 4, 1, generator=g, dtype=torch.float64) * 50, 0.0), base, atol=1e-11)
    assert torch.allclose(okl.kl_row_losses(a * 7.5, z, 0.0), base, atol=1e-12)
    # KL >= 0 (Gibbs).
    assert float(base.min()) >= -1e-14
    # d_logits sums to zero per row; d_attn is orthogonal to attn when eps = 0 (scale invariance).
    da, dz = okl.kl_loss_bwd(a, z, 1.0, eps=0.0)
    assert float(dz.sum(-1).abs().max()) < 1e-15
    assert float((da * a).sum(-1).abs().max()) < 1e-14


def test_kl_oracle_backward_matches_autograd_and_finite_differences():
    from oracle import kl_loss as okl

    g = torch.Generator().manual_seed(13)
    eps = 1e-3
    a = (torch.rand(2, 3, 9, generator=g, dtype=torch.float64) * torch.rand(2, 3, 1, generator=g, dtype=torch.float64))
    a[0, 1, :4] = 0.0  # zero mass entries, where log(p + eps) matters
    z = torch.randn(2, 3, 9, generator=g, dtype=torch.float64) * 2
    ag = a.clone().requires_grad_(True)
    zg = z.clone().requires_grad_(True)
    # autograd through the reference's torch formula (indexer_kl_fused.py:158-161)
    loss = okl.kl_loss_autograd(ag, zg, eps)
    assert abs(float(loss.detach()) - float(okl.kl_loss(a, z, eps))) < 1e-12
    (loss * 2.5).backward()
    da, dz = okl.kl_loss_bwd(a, z, 2.5, eps)
    torch.testing.assert_close(da, ag.grad, rtol=1e-10, atol=1e-13)
    # The reference's d_logits is gs * (softmax(z) - p) (indexer_kl_fused.py:152); the exact
    # derivative is gs * (softmax(z) * sum(p) - p) with sum(p) = S / (S + eps) < 1. The
    # oracle follows the reference; the difference is exactly gs * softmax(z) * (sum(p) - 1).
    gs = 2.5 / 6
    sum_p = (a / (a.sum(-1, keepdim=True) + eps)).sum(-1, keepdim=True)
    dz_exact = dz + gs * torch.softmax(z, -1) * (sum_p - 1)
    torch.testing.assert_close(dz_exact, zg.grad, rtol=1e-10, atol=1e-13)
    assert float((dz - zg.grad).abs().max()) > 1e-5  # the omitted factor is visible here
    # with eps = 0 the reference's formula is the exact gradient
    zg0 = z.clone().requires_grad_(True)
    p0 = a / a.sum(-1, keepdim=True)
    ((p0 * (torch.log(p0) .nan_to_num(neginf=0.0) - torch.log_softmax(zg0, -1))).sum(-1).mean() * 2.5).backward()
    torch.testing.assert_close(okl.kl_loss_bwd(a, z, 2.5, 0.0)[1], zg0.grad, rtol=1e-10, atol=1e-13)
    # central differences on a few coordinates
    h = 1e-6
    for idx in [(0, 0, 0), (0, 1, 2), (1, 2, 8)]:
        for t, d in ((a, da), (z, dz_exact)):
            tp, tm = t.clone(), t.clone()
            tp[idx] += h
            tm[idx] -= h
            args_p = (tp, z) if t is a else (a, tp)
            args_m = (tm, z) if t is a else (a, tm)
            fd = (float(okl.kl_loss(*args_p, eps)) - float(okl.kl_loss(*args_m, eps))) / (2 * h) * 2.5
            assert abs(fd - float(d[idx])) < 1e-6 * max(1.0, abs(fd))


def test_rope2d_oracle_identity_relative_position_and_brute_force():
    from oracle import layer_glue as olg

    g = torch.Generator().manual_seed(21)
    B, H, N, D = 1, 2, 6, 64
    t = torch.randn(B, H, N, D, generator=g, dtype=torch.float64).float()
    # position (0, 0) is the identity
    z = torch.zeros(B, N, 2, dtype=torch.long)
    torch.testing.assert_close(olg.rope2d(t, z), t, rtol=0, atol=0)
    # brute force over the reference's formula (rope.py:120-152): per 32-dim half with
    # position p and frequency f_i = 100^(-2i/32): out[i] = x[i] cos - x[i+16] sin,
    # out[i+16] = x[i+16] cos + x[i] sin
    pos = torch.randint(0, 40, (B, N, 2), generator=g)
    got = olg.rope2d(t, pos)
    for h in range(H):
        for n in range(N):
            for half, p in ((0, int(pos[0, n, 0])), (1, int(pos[0, n, 1]))):
                for i in range(16):
                    f = 1.0 / (100.0 ** (2 * i / 32))
                    c, s = math.cos(p * f), math.sin(p * f)
                    a, b = float(t[0, h, n, 32 * half + i]), float(t[0, h, n, 32 * half + 16 + i])
                    assert abs(float(got[0, h, n, 32 * half + i]) - (a * c - b * s)) < 1e-5
                    assert abs(float(got[0, h, n, 32 * half + 16 + i]) - (b * c + a * s)) < 1e-5
    # rotations preserve the norm, and scores depend only on position differences
    torch.testing.assert_close(got.norm(dim=-1), t.norm(dim=-1), rtol=1e-5, atol=1e-5)
    q = torch.randn(1, 1, 2, D, generator=g)
    k = torch.randn(1, 1, 2, D, generator=g)
    p1 = torch.tensor([[[3, 7], [5, 2]]])
    p2 = p1 + torch.tensor([[[4, 9]]])
    s1 = (olg.rope2d(q, p1)[0, 0, 0] * olg.rope2d(k, p1)[0, 0, 1]).sum()
    s2 = (olg.rope2d(q, p2)[0, 0, 0] * olg.rope2d(k, p2)[0, 0, 1]).sum()
    assert abs(float(s1) - float(s2)) < 1e-4


def test_pi3_rope2d_is_the_same_rotation_and_positions_match_the_grid():
    # Pi3's RoPE2D (pos_embed.py:112-160) against the brute-force-pinned VGGT rotation:
    # same frequencies (freq^(-2i/32) per 32-dim half), same halves (y then x), same
    # rotate_half pairing (i, i + 16) -- so one glue kernel serves both models. A slip in
    # either restatement (half order, pairing, frequency exponent) breaks the equality.
    from oracle import layer_glue as olg

    g = torch.Generator().manual_seed(22)
    t = torch.randn(2, 3, 50, 64, generator=g)
    pos = torch.randint(0, 38, (2, 50, 2), generator=g)
    torch.testing.assert_close(olg.rope2d_pi3(t, pos, 100.0), olg.rope2d(t, pos, 100.0), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(olg.rope2d_pi3(t, pos, 37.0), olg.rope2d(t, pos, 37.0), rtol=1e-6, atol=1e-6)
    # positions: 5 register tokens at (0, 0), then the (y, x) grid + 1 in row-major order
    p = olg.pi3_positions(2, 3, 4)
    assert p.shape == (2, 17, 2)
    assert p[0, :5].abs().sum() == 0
    assert p[0, 5].tolist() == [1, 1] and p[0, 6].tolist() == [1, 2] and p[0, 9].tolist() == [2, 1]
    assert p[1, -1].tolist() == [3, 4]


def test_layer_glue_oracle_matches_the_unfused_reference_order():
    # The fused projection (dsa_attention.py:583-625) equals the unfused path: qkv linear
    # -> reshape(B, N, 3, H, D) (:229-233), q_norm/k_norm, rope (:4935-4940); indexer
    # q_proj/k_proj/w_proj, k_norm, rope (indexer.py:302-320).
    from oracle import layer_glue as olg

    g = torch.Generator().manual_seed(22)
    B, N, dim, H, D, Hi = 1, 10, 128, 2, 64, 2
    x = torch.randn(B, N, dim, generator=g)
    qkv_w, qkv_b = torch.randn(3 * H * D, dim, generator=g) * 0.1, torch.randn(3 * H * D, generator=g)
    iq_w, ik_w, iw_w = (torch.randn(n, dim, generator=g) * 0.1 for n in (Hi * D, Hi * D, Hi))
    iq_b, ik_b, iw_b = (torch.randn(n, generator=g) for n in (Hi * D, Hi * D, Hi))
    lnp = {k: (torch.rand(D, generator=g) + 0.5, torch.randn(D, generator=g)) for k in ("q", "k", "idx_k")}
    pos = torch.randint(0, 12, (B, N, 2), generator=g)
    W = torch.cat([qkv_w, iq_w, ik_w, iw_w])
    bb = torch.cat([qkv_b, iq_b, ik_b, iw_b])
    q, k, v, iq, ik, iw = olg.fused_projection_glue(x, W, bb, dict(H=H, D=D, Hi=Hi, Di=D), lnp, pos)
    qkv = F.linear(x, qkv_w, qkv_b).reshape(B, N, 3, H, D).permute(2, 0, 3, 1, 4)
    rq, rk, rv = qkv.unbind(0)
    rq = F.layer_norm(rq, (D,), *lnp["q"], 1e-5)
    rk = F.layer_norm(rk, (D,), *lnp["k"], 1e-5)
    rq, rk = olg.rope2d(rq, pos), olg.rope2d(rk, pos)
    torch.testing.assert_close(q, rq.transpose(1, 2), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(k, rk.transpose(1, 2), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(v, rv.transpose(1, 2), rtol=1e-5, atol=1e-5)
    riq = F.linear(x, iq_w, iq_b).view(B, N, Hi, D)
    rik = F.layer_norm(F.linear(x, ik_w, ik_b).view(B, N, Hi, D), (D,), *lnp["idx_k"], 1e-5)
    rp = lambda t: olg.rope2d(t.permute(0, 2, 1, 3), pos).permute(0, 2, 1, 3)
    torch.testing.assert_close(iq, rp(riq), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ik, rp(rik), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(iw, F.linear(x, iw_w, iw_b), rtol=1e-5, atol=1e-5)
    # LayerNorm itself against a hand loop on one vector
    vec = F.linear(x, ik_w, ik_b).view(B, N, Hi, D)[0, 3, 1]
    mu = sum(float(a) for a in vec) / D
    var = sum((float(a) - mu) ** 2 for a in vec) / D
    want = [(float(a) - mu) / math.sqrt(var + 1e-5) * float(w) + float(b2)
            for a, w, b2 in zip(vec, *lnp["idx_k"])]
    got = F.layer_norm(vec, (D,), *lnp["idx_k"], 1e-5)
    assert max(abs(float(a) - b2) for a, b2 in zip(got, want)) < 1e-4


# ------------------------------------------------------------- source-downsample selector


def test_source_layout_tiny_case_by_hand():
    # 2 views of 2 special tokens + a 3 x 3 patch grid, factor 2: the pooled area is the
    # top-left 2 x 2 cell; the other 5 patches of a view are edge rows.
    from oracle import source_downsample as osd

    lay = osd.source_layout(11, 2, 2, 2)
    rows = [[t for t in r if t >= 0] for r in lay["source_to_fine"].tolist()]
    assert rows == [[0], [1], [11], [12],  # specials, view-major
                    [4], [7], [8], [9], [10], [15], [18], [19], [20], [21],  # edges, row-major per view
                    [2, 3, 5, 6], [13, 14, 16, 17]]  # one cell per view, (dy, dx) order
    assert (lay["special_count"], lay["edge_count"], lay["coarse_count"]) == (4, 10, 2)
    assert lay["expand_round_robin"] and lay["max_block_tokens"] == 4


@pytest.mark.parametrize("factor,rep", [(2, False), (3, False), (4, False), (4, True), (8, True)])
def test_source_layout_covers_each_token_once(factor, rep):
    from oracle import source_downsample as osd

    tpv, views, psi, grid = 5 + 37 * 37, 3, 5, 37
    lay = osd.source_layout(tpv, views, psi, factor, representative_points=rep)
    stf = lay["source_to_fine"]
    toks = stf[stf >= 0]
    assert len(set(toks.tolist())) == toks.size  # no token in two rows
    if not rep:
        assert sorted(toks.tolist()) == list(range(tpv * views))  # a partition of all tokens
        assert lay["max_block_tokens"] == factor * factor
    else:
        # representative points lie inside their own cell; specials and edges are complete
        off = lay["special_count"] + lay["edge_count"]
        cells = stf[off:]
        pooled = grid // factor * factor
        for r, row in enumerate(cells[: pooled // factor * pooled // factor]):
            cy, cx = divmod(r, pooled // factor)
            for t in row[row >= 0]:
                y, x = divmod(int(t) - psi, grid)
                assert cy * factor <= y < (cy + 1) * factor and cx * factor <= x < (cx + 1) * factor
        assert not lay["expand_round_robin"]
    assert lay["source_len"] == lay["special_count"] + lay["edge_count"] + lay["coarse_count"]


def test_source_pooling_equals_avg_pool2d_and_copies():
    from oracle import source_downsample as osd

    g = torch.Generator().manual_seed(5)
    tpv, views, psi, grid, f = 5 + 9 * 9, 2, 5, 9, 2
    k = torch.randn(1, tpv * views, 2, 64, generator=g).bfloat16()
    w = (1 + 0.3 * torch.randn(1, tpv * views, 2, generator=g)).bfloat16()
    lay = osd.source_layout(tpv, views, psi, f)
    sk, sw = osd.pool_sources(k, w, lay)
    img = k.float().view(views, tpv, 128)[:, psi:].reshape(views, grid, grid, 128).permute(0, 3, 1, 2)
    ref = F.avg_pool2d(img[:, :, :8, :8], f).permute(0, 2, 3, 1).reshape(-1, 2, 64).bfloat16()
    off = lay["special_count"] + lay["edge_count"]
    assert torch.equal(sk[0, off:], ref)
    imgw = w.float().view(views, tpv, 2)[:, psi:].reshape(views, grid, grid, 2).permute(0, 3, 1, 2)
    refw = F.avg_pool2d(imgw[:, :, :8, :8], f).permute(0, 2, 3, 1).reshape(-1, 2).bfloat16()
    assert torch.equal(sw[0, off:], refw)
    single = torch.from_numpy(lay["source_to_fine"][:off, 0])
    assert torch.equal(sk[0, :off], k[0, single]) and torch.equal(sw[0, :off], w[0, single])


def test_source_coarse_budget_by_hand():
    from oracle import source_downsample as osd

    # VGGT at S = 32, factor 2: 160 specials, 73 edges x 32, 324 cells x 32; 43968 tokens over
    # 12864 rows -> ceil(1024 / 3.41791 * 1.1) = 330.
    lay = osd.source_layout(1374, 32, 5, 2)
    assert (lay["source_len"], osd.coarse_topk(lay, 1024)) == (12864, 330)
    # Specials (160) outnumber the budget (ceil(256 / 7.667 * 1.1) = 37): 160 + ceil(96 / 16 * 1.1).
    lay = osd.source_layout(20 + 16 * 16, 8, 20, 4)
    assert osd.coarse_topk(lay, 256) == 160 + 7
    assert osd.coarse_topk(lay, 256, explicit=10**6) == lay["source_len"]


def test_source_expand_by_hand():
    from oracle import source_downsample as osd

    lay = osd.source_layout(11, 2, 2, 2)  # rows as in the tiny case above
    c = torch.tensor([[[14, 0, 15]]])
    # round robin: m = 0 -> 2, 0, 13; m = 1 -> 3, (special has one token), 14; m = 2 -> 5, 16; m = 3 -> 6, 17
    assert osd.expand(c, lay, 6, 22).tolist() == [[[2, 0, 13, 3, 14, 5]]]
    # 9 valid tokens for a target of 12: repeat the last min(9, 4) = 4 cyclically
    assert osd.expand(c, lay, 12, 22, pad_window=4).tolist() == [[[2, 0, 13, 3, 14, 5, 16, 6, 17, 5, 16, 6]]]
    # row-by-row order (representative points)
    lay_rep = osd.source_layout(2 + 8 * 8, 1, 2, 8, representative_points=True)
    r0 = lay_rep["special_count"] + lay_rep["edge_count"]
    got = osd.expand(torch.tensor([[[r0, 1]]]), lay_rep, 5, 66)[0, 0].tolist()
    cell = [t for t in lay_rep["source_to_fine"][r0].tolist() if t >= 0]
    assert got == cell + [1]


def test_source_order_by_score_by_hand():
    from oracle import source_downsample as osd

    c = torch.tensor([[[5, 3, 9, 1]]])
    s = torch.tensor([[[1.0, 2.0, 1.0, 2.0]]])
    assert osd.order_by_score(c, s).tolist() == [[[1, 3, 5, 9]]]


def test_sparse_attention_non_finite_scores_follow_the_reference_softmax():
    # An inf in a selected K row gives a +inf score: the reference's softmax
    # (tests/sparse_index_flash_attn_tests.py:66, dsa_attention.py:4747) makes that (t, h)
    # row nan; an all-invalid row is zeroed by the masked_fill. Pinned against the same ops
    # written out on one row.
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 3, 2, 4, generator=g)
    k = torch.randn(1, 5, 2, 4, generator=g)
    v = torch.randn(1, 5, 2, 4, generator=g)
    q[0, 0, 1] = 1.0
    k[0, 2, 1, 0] = float("inf")           # score of (t=0, h=1, key 2) is +inf
    pos = torch.tensor([[[0, 2, 4], [1, 3, 4], [-1, -1, -1]]], dtype=torch.int32)
    o, attn, lse = oatt.sparse_attention(q, k, v, pos, 0.5)
    assert torch.isnan(o[0, 0, 1]).all() and torch.isfinite(o[0, 0, 0]).all()
    assert lse[0, 0, 1] == float("inf") and torch.isfinite(o[0, 1]).all()
    assert torch.equal(o[0, 2], torch.zeros(2, 4)) and torch.equal(attn[0, 2], torch.zeros(3))
    s = (q[0, 1, 0] * k[0, [1, 3, 4], 0]).sum(-1) * 0.5
    torch.testing.assert_close(o[0, 1, 0], torch.softmax(s, 0) @ v[0, [1, 3, 4], 0])
