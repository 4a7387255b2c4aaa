"""Tie-aware comparison of a top-k index set against the fp32 oracle.

Test infrastructure only (see ``oracle/__init__.py``).

Contract (from the parity bar of this path): indices are compared as sets (the reference
returns ``sorted=False`` results, ``sparse_topk_indexer.py:1311``); they must be
bit-exact, except where the reference fp32 scores tie within 1e-6 relative. With
tau = the k-th largest oracle score of the row, every index in the symmetric difference
of the two sets must have an oracle score within ``rtol * |tau|`` of tau.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class TopkReport:
    rows: int
    rows_exact: int          # rows whose set equals the oracle set bit for bit
    rows_tie_swapped: int    # rows that differ only inside the tie window
    bad_rows: int            # rows that violate the contract
    first_bad: str = ""

    @property
    def ok(self) -> bool:
        return self.bad_rows == 0


def check_topk_rows(
    ref_scores: torch.Tensor,
    got_idx: torch.Tensor,
    topk: int,
    rtol: float = 1e-6,
) -> TopkReport:
    """Check got_idx [R, K] against full oracle score rows ref_scores [R, S] (fp32).

    Conditions per row: K distinct indices in [0, S); every index whose oracle score
    exceeds tau by more than the window is present; every returned index has an oracle
    score no lower than tau minus the window.
    """
    ref_scores = ref_scores.float()
    rows, src_len = ref_scores.shape
    kk = min(int(topk), src_len)
    got = got_idx.long()
    assert got.shape == (rows, kk), (tuple(got.shape), rows, kk)
    tau = ref_scores.topk(kk, dim=-1).values[:, -1]  # k-th largest
    win = rtol * tau.abs()
    in_range = ((got >= 0) & (got < src_len)).all(dim=-1)
    safe = got.clamp(0, src_len - 1)
    srt = safe.sort(dim=-1).values
    distinct = (srt[:, 1:] != srt[:, :-1]).all(dim=-1) if kk > 1 else torch.ones(rows, dtype=torch.bool)
    got_scores = ref_scores.gather(1, safe)
    low_ok = (got_scores >= (tau - win).unsqueeze(-1)).all(dim=-1)
    member = torch.zeros((rows, src_len), dtype=torch.bool)
    member.scatter_(1, safe, True)
    must = ref_scores > (tau + win).unsqueeze(-1)
    high_ok = ~(must & ~member).any(dim=-1)
    ok = in_range & distinct & low_ok & high_ok
    ref_set = torch.zeros((rows, src_len), dtype=torch.bool)
    ref_set.scatter_(1, ref_scores.topk(kk, dim=-1).indices, True)
    exact = (ref_set == member).all(dim=-1) & ok
    bad = (~ok).nonzero().flatten()
    first = ""
    if bad.numel():
        r = int(bad[0])
        first = (
            f"row {r}: in_range={bool(in_range[r])} distinct={bool(distinct[r])} "
            f"low_ok={bool(low_ok[r])} high_ok={bool(high_ok[r])} tau={float(tau[r])!r}"
        )
    return TopkReport(
        rows=rows,
        rows_exact=int(exact.sum()),
        rows_tie_swapped=int((ok & ~exact).sum()),
        bad_rows=int((~ok).sum()),
        first_bad=first,
    )
