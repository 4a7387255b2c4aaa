"""Writes the small golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Every expected value here is computed with plain Python float (fp64) loops written
directly from the mathematical definition, independently of the oracle code, so the
fixtures can pin the oracle:

* indexer_kat.json - the hand-checkable indexer top-k case of the reference test
  ``tests/indexer_projected_tests.py:130-187`` (q = [[1,0],[0,1]],
  k = [[1,0],[0.2,0.8],[0,1],[0.8,0.2]], w = 1, top-2, scale = 1/sqrt(2)) with the view
  bias removed; plus a 2-head case with signed w and an additive mask (-inf entries).
* indexer_view_bias_kat.json - the reference's view-bias cases of
  ``tests/indexer_projected_tests.py``: the top-2 case of :130-187 with its view bias, the
  all-tie top-1 case of :64-128 (q = k = 0, so the bias alone ranks the keys) and the
  gradient case of :189-243 with the table gradient of sum(topk_scores) counted by hand
  from its (unambiguous) top-2 sets; plus a 2-head case with a mask and 3 x 2 views.
* attn_fixture.json - sparse attention with the reference's hard-coded top-k index
  fixture ``[[0,2,5],[1,4,3],[0,3,5],[2,4,1]]`` (``tests/dsa_objective_value_gate_tests.py:370-374``)
  and a ragged row with -1 padding (``tests/sparse_index_flash_attn_tests.py:37-44``):
  o, attn_sum, lse and the gradients dq, dk, dv for a fixed dO and dattn.
"""
from __future__ import annotations

import json
import math
import random
from pathlib import Path

HERE = Path(__file__).resolve().parent


def relu(x):
    return x if x > 0 else 0.0


def indexer_scores_bf(q, k, w, scale, mask=None):
    # q[t][h][d], k[s][h][d], w[s][h]
    out = []
    for t in range(len(q)):
        row = []
        for s in range(len(k)):
            acc = 0.0
            for h in range(len(q[t])):
                z = sum(q[t][h][d] * k[s][h][d] for d in range(len(q[t][h])))
                acc += w[s][h] * relu(scale * z)
            if mask is not None:
                acc += mask[t][s]
            row.append(acc)
        out.append(row)
    return out


def topk_set(row, kk):
    order = sorted(range(len(row)), key=lambda i: (-row[i], i))
    return sorted(order[:kk])


def make_indexer_kat():
    cases = []
    q = [[[1.0, 0.0]], [[0.0, 1.0]]]
    k = [[[1.0, 0.0]], [[0.2, 0.8]], [[0.0, 1.0]], [[0.8, 0.2]]]
    w = [[1.0], [1.0], [1.0], [1.0]]
    scale = 1.0 / math.sqrt(2.0)
    sc = indexer_scores_bf(q, k, w, scale)
    cases.append(dict(name="reference_projected_tests_no_view_bias", q=q, k=k, w=w, mask=None,
                      topk=2, scale=scale, scores=sc, expected_sets=[topk_set(r, 2) for r in sc]))
    rng = random.Random(20261201)
    T, S, H, D = 3, 7, 2, 3
    q2 = [[[rng.choice([-1.0, -0.5, 0.5, 1.0, 2.0]) for _ in range(D)] for _ in range(H)] for _ in range(T)]
    k2 = [[[rng.choice([-1.0, 0.25, 0.5, 1.5]) for _ in range(D)] for _ in range(H)] for _ in range(S)]
    w2 = [[rng.choice([-0.5, 0.75, 1.0, 1.25]) for _ in range(H)] for _ in range(S)]
    mask = [[(-math.inf if (t + s) % 5 == 0 else 0.125 * ((t * 3 + s) % 4)) for s in range(S)] for t in range(T)]
    sc2 = indexer_scores_bf(q2, k2, w2, 0.5, mask)
    cases.append(dict(name="two_heads_signed_w_mask", q=q2, k=k2, w=w2, mask=mask, topk=3, scale=0.5,
                      scores=sc2, expected_sets=[topk_set(r, 3) for r in sc2]))
    return cases


def make_view_bias_kat():
    def case(name, q, k, w, qv, sv, table, topk, scale, mask=None, grad=False):
        sc = indexer_scores_bf(q, k, w, scale, mask)
        sc = [[sc[t][s] + table[qv[t]][sv[s]] for s in range(len(k))] for t in range(len(q))]
        c = dict(name=name, q=q, k=k, w=w, mask=mask, q_view_ids=[qv], s_view_ids=[sv], view_bias=[table],
                 topk=topk, scale=scale, scores=sc)
        if grad:
            # d sum(topk_scores) / d table: one per selected (t, s), at (q_view[t], s_view[s])
            g = [[0.0] * len(table[0]) for _ in table]
            for t, row in enumerate(sc):
                for s in topk_set(row, topk):
                    g[qv[t]][sv[s]] += 1.0
            c["table_grad_of_sum"] = [g]
        return c

    cases = []
    scale = 1.0 / math.sqrt(2.0)
    cases.append(case("reference_view_bias_top2",
                      [[[1.0, 0.0]], [[0.0, 1.0]]],
                      [[[1.0, 0.0]], [[0.2, 0.8]], [[0.0, 1.0]], [[0.8, 0.2]]],
                      [[1.0]] * 4, [0, 1], [0, 0, 1, 1], [[0.0, 4.0], [3.0, 0.0]], 2, scale))
    cases.append(case("reference_view_bias_ties_top1",
                      [[[0.0] * 4], [[0.0] * 4]], [[[0.0] * 4]] * 4, [[1.0]] * 4,
                      [0, 1], [0, 0, 1, 1], [[0.0, 5.0], [7.0, 0.0]], 1, 0.5))
    cases.append(case("reference_view_bias_gradient",
                      [[[1.0, 0.0]], [[0.0, 1.0]]],
                      [[[1.0, 0.0]], [[0.0, 1.0]], [[0.7, 0.3]], [[0.3, 0.7]]],
                      [[1.0]] * 4, [0, 1], [0, 0, 1, 1], [[0.0, 2.0], [1.5, 0.0]], 2, scale, grad=True))
    rng = random.Random(20261202)
    T, S, H, D = 4, 9, 2, 3
    q2 = [[[rng.choice([-1.0, -0.5, 0.5, 1.0, 2.0]) for _ in range(D)] for _ in range(H)] for _ in range(T)]
    k2 = [[[rng.choice([-1.0, 0.25, 0.5, 1.5]) for _ in range(D)] for _ in range(H)] for _ in range(S)]
    w2 = [[rng.choice([-0.5, 0.75, 1.0, 1.25]) for _ in range(H)] for _ in range(S)]
    mask = [[(-math.inf if (t + 2 * s) % 7 == 0 else 0.25 * ((t + s) % 3)) for s in range(S)] for t in range(T)]
    qv = [0, 2, 1, 2]
    sv = [1, 0, 0, 1, 1, 0, 1, 0, 1]
    table = [[0.5, -1.0], [2.0, 0.0], [-0.75, 1.5]]
    cases.append(case("two_heads_mask_three_by_two_views", q2, k2, w2, qv, sv, table, 3, 0.5, mask, grad=True))
    return cases


def attention_bf(q, k, v, pos, scale, do, dattn):
    """fp64 brute force of o, attn_sum, lse and (dq, dk, dv) for loss = <o,dO> + <attn_sum,dattn>."""
    T, H, D = len(q), len(q[0]), len(q[0][0])
    S = len(k)
    K = len(pos[0])
    o = [[[0.0] * D for _ in range(H)] for _ in range(T)]
    asum = [[0.0] * K for _ in range(T)]
    lse = [[-math.inf] * H for _ in range(T)]
    dq = [[[0.0] * D for _ in range(H)] for _ in range(T)]
    dk = [[[0.0] * D for _ in range(H)] for _ in range(S)]
    dv = [[[0.0] * D for _ in range(H)] for _ in range(S)]
    for t in range(T):
        valid = [0 <= pos[t][j] < S for j in range(K)]
        for h in range(H):
            s = [scale * sum(q[t][h][d] * k[pos[t][j]][h][d] for d in range(D)) if valid[j] else None
                 for j in range(K)]
            vals = [x for x in s if x is not None]
            if not vals:
                continue
            mx = max(vals)
            z = sum(math.exp(x - mx) for x in vals)
            lse[t][h] = mx + math.log(z)
            p = [math.exp(s[j] - lse[t][h]) if valid[j] else 0.0 for j in range(K)]
            for j in range(K):
                asum[t][j] += p[j]
                if valid[j]:
                    for d in range(D):
                        o[t][h][d] += p[j] * v[pos[t][j]][h][d]
            # d loss / d p_j = dO . v_j + dattn_j ; softmax backward
            g = [(sum(do[t][h][d] * v[pos[t][j]][h][d] for d in range(D)) + dattn[t][j]) if valid[j] else 0.0
                 for j in range(K)]
            gbar = sum(p[j] * g[j] for j in range(K))
            for j in range(K):
                if not valid[j]:
                    continue
                ds = p[j] * (g[j] - gbar)  # d loss / d s_j
                sj = pos[t][j]
                for d in range(D):
                    dq[t][h][d] += scale * ds * k[sj][h][d]
                    dk[sj][h][d] += scale * ds * q[t][h][d]
                    dv[sj][h][d] += p[j] * do[t][h][d]
    return o, asum, lse, dq, dk, dv


def make_attention_fixture():
    rng = random.Random(123)
    T, S, H, D = 5, 6, 2, 4
    q = [[[rng.gauss(0, 1) for _ in range(D)] for _ in range(H)] for _ in range(T)]
    k = [[[rng.gauss(0, 1) for _ in range(D)] for _ in range(H)] for _ in range(S)]
    v = [[[rng.gauss(0, 1) for _ in range(D)] for _ in range(H)] for _ in range(S)]
    do = [[[rng.gauss(0, 1) for _ in range(D)] for _ in range(H)] for _ in range(T)]
    pos = [[0, 2, 5], [1, 4, 3], [0, 3, 5], [2, 4, 1], [3, -1, -1]]
    dattn = [[rng.gauss(0, 1) for _ in range(3)] for _ in range(T)]
    scale = 0.5
    o, asum, lse, dq, dk, dv = attention_bf(q, k, v, pos, scale, do, dattn)
    return dict(q=q, k=k, v=v, do=do, kv_positions=pos, dattn=dattn, scale=scale,
                o=o, attn_sum=asum, lse=lse, dq=dq, dk=dk, dv=dv)


def main():
    (HERE / "indexer_kat.json").write_text(json.dumps(make_indexer_kat(), indent=1) + "\n")
    (HERE / "indexer_view_bias_kat.json").write_text(json.dumps(make_view_bias_kat(), indent=1) + "\n")
    (HERE / "attn_fixture.json").write_text(json.dumps(make_attention_fixture(), indent=1) + "\n")
    print("wrote", HERE / "indexer_kat.json", HERE / "indexer_view_bias_kat.json", HERE / "attn_fixture.json")


if __name__ == "__main__":
    main()
