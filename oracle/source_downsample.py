"""CPU restatement of the source-downsample coarse selector ("legacy" strategy).

Test infrastructure only (see ``oracle/__init__.py``).

An approximate top-k for long inputs, used only at inference: the keys of each view's
patch grid are average-pooled over ``factor x factor`` cells (special tokens and the edge
tokens outside the pooled area stay as they are), the indexer picks the top
``coarse_topk`` of these source rows, and every chosen source row is expanded back to the
fine tokens it covers. Reference: ``easyvolcap/official_vggt/layers/dsa_attention.py``

* ``source_layout``: ``_get_source_downsample_layout`` ``:3069-3259`` (+ ``_infer_patch_grid``
  ``:3034-3042``) without the factor >= 4 sub-cell tables, which only the non-legacy
  strategies read;
* ``pool_sources``: ``_prepare_source_downsample_projected`` ``:3386-3457,3519`` (special
  rows copied, edge rows gathered, ``F.avg_pool2d`` or the representative-point mean for
  the coarse rows, concatenated in that order);
* ``coarse_topk``: ``_resolve_source_downsample_coarse_topk`` ``:3328-3375`` for the legacy
  strategy, ``_get_source_downsample_effective_avg_expand`` ``:3290-3296``;
* ``expand``: ``_expand_source_downsample_chunk`` ``:4079-4128`` with the pad window of
  ``_resolve_source_downsample_pad_window`` ``:3377-3384``;
* ``select``: the legacy branch of ``_select_topk_source_downsample_chunk`` ``:4187-4217``,
  the coarse top-k being the oracle indexer's ``scores.topk(sorted=False)``;
* ``order_by_score``: the order in which this build expands the chosen rows (score
  descending, row ascending), one fixed choice for the reference's unspecified order.

The pooled keys are computed as the reference's torch ops do for 16-bit inputs: an fp32
sum over the cell in row-major order (or the representative points in their listed
order), divided by the count, rounded once to the input dtype.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import indexer as oidx


def infer_patch_grid(image_tokens_per_view: int, grid_h: int = 0, grid_w: int = 0) -> Tuple[int, int]:
    """reference: dsa_attention.py:3034-3042"""
    if grid_h > 0 and grid_w > 0 and grid_h * grid_w == image_tokens_per_view:
        return grid_h, grid_w
    side = math.isqrt(max(int(image_tokens_per_view), 0))
    if side > 0 and side * side == image_tokens_per_view:
        return side, side
    return 0, 0


def representative_offsets(factor: int, representative_points: bool):
    """Cell offsets a coarse row covers (reference: dsa_attention.py:3108-3122)."""
    if not (factor > 2 and representative_points):
        return [(yy, xx) for yy in range(factor) for xx in range(factor)], True
    quarter = max(factor // 4, 0)
    low = min(max(quarter, 0), factor - 1)
    high = max(min(factor - 1 - quarter, factor - 1), 0)
    offs = []
    for item in ((low, low), (low, high), (high, low), (high, high)):
        if item not in offs:
            offs.append(item)
    return offs, False


def source_layout(tokens_per_view: int, num_views: int, patch_start_idx: int, factor: int,
                  grid_h: int = 0, grid_w: int = 0, representative_points: bool = False) -> Optional[Dict]:
    """Source rows and the fine tokens each covers (reference: dsa_attention.py:3069-3259).

    Rows: the special tokens of every view (view-major), then per view the image tokens
    outside the pooled ``(grid_h // f * f) x (grid_w // f * f)`` area in row-major order,
    then per view the coarse cells in row-major order. ``source_to_fine[r, m]`` is the
    m-th fine token of row r (-1 past the row's count).
    """
    factor = max(int(factor), 1)
    if tokens_per_view <= 0 or num_views <= 0:
        return None
    if patch_start_idx < 0 or patch_start_idx >= tokens_per_view:
        return None
    image = tokens_per_view - patch_start_idx
    gh, gw = infer_patch_grid(image, grid_h, grid_w)
    if gh <= 0 or gw <= 0:
        return None
    offs, round_robin = representative_offsets(factor, representative_points)
    M = len(offs)
    ph, pw = (gh // factor) * factor, (gw // factor) * factor
    ch, cw = ph // factor, pw // factor
    rows = []
    for v in range(num_views):
        for i in range(patch_start_idx):
            rows.append([v * tokens_per_view + i])
    special_count = len(rows)
    for v in range(num_views):
        base = v * tokens_per_view + patch_start_idx
        for y in range(gh):
            for x in range(gw):
                if y < ph and x < pw:
                    continue
                rows.append([base + y * gw + x])
    edge_count = len(rows) - special_count
    for v in range(num_views):
        base = v * tokens_per_view + patch_start_idx
        for cy in range(ch):
            for cx in range(cw):
                toks = []
                for yy, xx in offs:
                    y, x = cy * factor + yy, cx * factor + xx
                    if y < gh and x < gw:
                        toks.append(base + y * gw + x)
                rows.append(toks)
    coarse_count = len(rows) - special_count - edge_count
    L = len(rows)
    stf = np.full((L, M), -1, dtype=np.int64)
    for r, toks in enumerate(rows):
        stf[r, :len(toks)] = toks
    mapped = special_count + edge_count + coarse_count * M
    non_special = L - special_count
    return dict(
        tokens_per_view=tokens_per_view, num_views=num_views, patch_start_idx=patch_start_idx,
        grid_h=gh, grid_w=gw, factor=factor, pooled_h=ph, pooled_w=pw, coarse_h=ch, coarse_w=cw,
        special_count=special_count, edge_count=edge_count, coarse_count=coarse_count,
        source_len=L, max_block_tokens=M, expand_round_robin=round_robin,
        source_to_fine=stf, source_valid=stf >= 0,
        avg_expand_tokens=mapped / L,
        non_special_source_len=non_special,
        non_special_avg_expand_tokens=(mapped - special_count) / non_special if non_special > 0 else 0.0,
    )


def pool_sources(k: torch.Tensor, w: torch.Tensor, layout: Dict) -> Tuple[torch.Tensor, torch.Tensor]:
    """Source keys and gates ``[B, L, Hi, Di]``, ``[B, L, Hi]`` in the input dtype: each
    source row is the mean of its fine rows, fp32 sum in listed order, divided by the
    count and rounded once (reference: dsa_attention.py:3412-3457,3519-3520)."""
    stf = torch.from_numpy(layout["source_to_fine"])
    valid = stf >= 0
    cnt = valid.sum(-1).to(torch.float32)
    idx = stf.clamp(min=0)
    kf, wf = k.float(), w.float()
    sk = torch.zeros(k.shape[0], stf.shape[0], *k.shape[2:], dtype=torch.float32)
    sw = torch.zeros(w.shape[0], stf.shape[0], w.shape[2], dtype=torch.float32)
    for m in range(stf.shape[1]):
        vm = valid[:, m].to(torch.float32)
        sk += kf[:, idx[:, m]] * vm.view(1, -1, 1, 1)
        sw += wf[:, idx[:, m]] * vm.view(1, -1, 1)
    sk = sk / cnt.view(1, -1, 1, 1)
    sw = sw / cnt.view(1, -1, 1)
    return sk.to(k.dtype), sw.to(w.dtype)


def coarse_topk(layout: Dict, topk: int, coarse_ratio: float = 1.1, explicit: int = 0) -> int:
    """Source rows to select (reference: dsa_attention.py:3328-3375, legacy strategy)."""
    ct = int(explicit or 0)
    if ct <= 0:
        ratio = max(float(coarse_ratio or 1.1), 1.0)
        avg = max(float(layout["avg_expand_tokens"]), 1.0)
        ct = int(math.ceil((float(topk) / avg) * ratio))
        special = min(int(layout["special_count"]), int(topk))
        ns_len = int(layout["non_special_source_len"])
        ns_avg = max(float(layout["non_special_avg_expand_tokens"]), 1.0)
        if special > 0 and special < int(topk) and ct < special and ns_len > 0:
            budget = int(math.ceil((float(int(topk) - special) / max(ns_avg, 1.0)) * ratio))
            ct = max(ct, special + max(budget, 1))
    return min(max(int(ct), 1), int(layout["source_len"]))


def expand(coarse_indices: torch.Tensor, layout: Dict, topk: int, fine_src_len: int,
           pad_window: int = 64) -> torch.Tensor:
    """Fine token indices ``[B, T, min(topk, fine_src_len)]`` (int64) from source-row
    indices ``[B, T, Kc]`` in their given order (reference: dsa_attention.py:4079-4128).

    Round robin (full cells): the m-th token of every chosen row, m = 0, 1, ...; else
    row by row. Valid tokens are compacted in that order and cut to the target; a row
    with fewer valid tokens repeats its last ``min(count, pad_window)`` ones cyclically.
    """
    stf = torch.from_numpy(layout["source_to_fine"])
    valid = stf >= 0
    B, T, Kc = coarse_indices.shape
    M = stf.shape[1]
    target = min(int(topk), int(fine_src_len))
    blocks = stf[coarse_indices.reshape(-1).long()].reshape(B, T, Kc, M)
    bvalid = valid[coarse_indices.reshape(-1).long()].reshape(B, T, Kc, M)
    if layout["expand_round_robin"]:
        flat = blocks.permute(0, 1, 3, 2).reshape(B, T, Kc * M)
        fvalid = bvalid.permute(0, 1, 3, 2).reshape(B, T, Kc * M)
    else:
        flat = blocks.reshape(B, T, Kc * M)
        fvalid = bvalid.reshape(B, T, Kc * M)
    if flat.shape[-1] < target:
        # Fewer slots than the target (Kc * M < target): the reference's torch.where then
        # fails on mismatched shapes; here the list is read as if extended by empty slots,
        # so such rows are padded like any row short of valid tokens.
        fill = target - flat.shape[-1]
        flat = torch.cat([flat, flat.new_full((B, T, fill), -1)], -1)
        fvalid = torch.cat([fvalid, fvalid.new_zeros((B, T, fill))], -1)
    rank = fvalid.to(torch.int64).cumsum(-1) - 1
    invalid_rank = flat.shape[-1] + torch.arange(flat.shape[-1], dtype=torch.int64).view(1, 1, -1)
    order = torch.argsort(torch.where(fvalid, rank, invalid_rank), dim=-1)
    compact = flat.gather(-1, order[..., :target])
    counts = fvalid.sum(-1).clamp(max=target)
    if bool((counts < target).any()):
        safe = counts.clamp(min=1)
        keep = torch.arange(target, dtype=torch.int64).view(1, 1, -1)
        window = torch.minimum(safe, torch.full_like(safe, max(1, min(int(pad_window), target))))
        start = safe - window
        offs = (keep - safe.unsqueeze(-1)).clamp_min(0)
        rep = start.unsqueeze(-1) + torch.remainder(offs, window.unsqueeze(-1))
        compact = torch.where(keep < safe.unsqueeze(-1), compact, compact.gather(-1, rep))
    return compact


def order_by_score(coarse_indices: torch.Tensor, coarse_scores: torch.Tensor) -> torch.Tensor:
    """The chosen rows by score descending, row index ascending on ties: the order this
    build expands in. The reference expands in the order of an unsorted torch.topk
    (indexer.py:600-603), which is unspecified; this fixes one."""
    idx = coarse_indices.long()
    by_idx = idx.sort(dim=-1, stable=True)
    sc = coarse_scores.float().gather(-1, by_idx.indices)
    by_score = (-sc).sort(dim=-1, stable=True)
    return by_idx.values.gather(-1, by_score.indices)


def select(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, layout: Dict, topk: int,
           softmax_scale: float, coarse_ratio: float = 1.1, pad_window: int = 64,
           coarse_indices: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(fine indices, coarse indices) of the legacy selector. ``coarse_indices`` given:
    expand those (in their order) instead of selecting them from the oracle scores."""
    sk, sw = pool_sources(k, w, layout)
    kc = coarse_topk(layout, topk, coarse_ratio)
    if coarse_indices is None:
        scores = oidx.indexer_scores(q, sk, sw, None, softmax_scale)
        coarse_indices = scores.topk(min(kc, scores.shape[-1]), dim=-1, sorted=False)[1]
    fine_len = layout["tokens_per_view"] * layout["num_views"]
    return expand(coarse_indices, layout, topk, fine_len, pad_window), coarse_indices


# ------------------------------------------------------------------ the other strategies
#
# * ``resolve_strategy``: ``_resolve_source_downsample_strategy`` ``:3273-3288``;
# * ``coarse_topk_for``: ``_resolve_source_downsample_coarse_topk`` ``:3328-3375`` with the
#   sub-cell expansion of ``_get_source_downsample_effective_avg_expand`` ``:3290-3296``;
# * ``subcell_table`` / ``pool_rows``: the factor-4 sub-cell tables and 2 x 2 pooled keys of
#   ``:3229-3257`` and ``:3458-3504`` (``_get_source_downsample_subcell_group_ids``
#   ``:3617-3627``);
# * ``static_pack4_table``: ``:3521-3542``; ``expand`` with a per-batch table:
#   ``_expand_source_downsample_chunk_batched`` ``:4129-4186``;
# * ``rerank``: ``_select_source_downsample_exact_rerank`` ``:3599-3635`` with the candidate
#   scores of ``_score_source_downsample_candidates`` ``:3554-3597``;
# * ``subcell_top1``: ``_select_source_downsample_subcell_top1`` ``:3629-3812``;
# * ``query_downsample`` / ``qk_sym_x2``: ``_prepare_query_downsample_chunk`` ``:3929-3997``,
#   ``_broadcast_source_downsample_chunk_to_queries`` ``:3999-4017`` and
#   ``_select_source_downsample_qk_sym_x2_*`` ``:4019-4078``;
# * ``select_strategy``: ``_select_topk_source_downsample_chunk`` ``:4187-4260`` (retry
#   growth and the full-indexer fallback).
#
# Candidate and sub-cell scores are the indexer's fp32 formula (``oracle.indexer``); the
# reference evaluates them with torch ops in the 16-bit input dtype, so its ranking is
# that of bf16/fp16-rounded scores, with ties broken by an unsorted torch.topk.

STRATEGIES = ("legacy", "exact_rerank", "subcell_top1", "subcell_static_pack4", "qk_sym_x2_broadcast")


def resolve_strategy(strategy: Optional[str], factor: int) -> str:
    """reference: dsa_attention.py:3273-3288"""
    s = str(strategy or "legacy").strip().lower()
    f = int(factor)
    if s == "qk_sym_x2_broadcast":
        return s if f == 2 else "legacy"
    if f < 4 and s != "legacy":
        return "legacy"
    if s not in STRATEGIES:
        return "legacy"
    return s


def coarse_topk_for(layout: Dict, topk: int, strategy: str, coarse_ratio: float = 1.1, explicit: int = 0) -> int:
    """Source rows to select for a strategy (reference: dsa_attention.py:3328-3375)."""
    if int(explicit or 0) > 0 or strategy not in ("subcell_top1", "subcell_static_pack4"):
        return coarse_topk(layout, topk, coarse_ratio, explicit)
    ratio = max(float(coarse_ratio or 1.1), 1.0)
    f = int(layout["factor"])
    L = int(layout["source_len"])
    special = min(int(layout["special_count"]), int(topk))
    if strategy == "subcell_static_pack4":
        pack = max(f // 2, 1) ** 2
        ct = int(special + math.ceil((float(max(int(topk) - special, 0)) / float(max(pack, 1))) * ratio))
        return min(max(ct, 1), L)
    per_block = max(f // 2, 1) ** 2
    mapped = int(layout["special_count"]) + int(layout["edge_count"]) + int(layout["coarse_count"]) * per_block
    avg = max(float(mapped) / float(max(L, 1)), 1.0)
    ct = int(math.ceil((float(topk) / avg) * ratio))
    ns_len = int(layout["non_special_source_len"])
    ns_avg = max(float(layout["non_special_avg_expand_tokens"]), 1.0)
    ns_avg = max(ns_avg / float(max(f, 1) / 2.0) ** 2, 1.0)
    if special > 0 and special < int(topk) and ct < special and ns_len > 0:
        budget = int(math.ceil((float(int(topk) - special) / max(ns_avg, 1.0)) * ratio))
        ct = max(ct, special + max(budget, 1))
    return min(max(int(ct), 1), L)


def subcell_table(layout: Dict) -> Optional[np.ndarray]:
    """Tokens of the 2 x 2 sub-cells of every coarse cell, int64 ``[C, 4, 4]``: sub-cell
    g = 2 sy + sx covers the cell offsets (yy, xx) with yy // 2 = sy and xx // 2 = sx, in
    their (yy, xx) order (reference: dsa_attention.py:3229-3257, :3617-3627). Only for
    factor 4 without representative points: the reference's 2 x 2 pooled keys reshape only
    then (:3478-3504); with representative points it has no sub-cell keys."""
    if int(layout["factor"]) != 4 or not layout["expand_round_robin"]:
        return None
    off = int(layout["special_count"]) + int(layout["edge_count"])
    C = int(layout["coarse_count"])
    cells = layout["source_to_fine"][off:off + C]  # [C, 16], offsets (yy, xx) row-major
    groups = [[yy * 4 + xx for yy in range(4) for xx in range(4) if (yy // 2) * 2 + xx // 2 == g] for g in range(4)]
    return np.stack([cells[:, pos] for pos in groups], axis=1)


def pool_rows(k: torch.Tensor, w: Optional[torch.Tensor], table: np.ndarray, round_sum: bool = False):
    """Mean of the listed rows of ``k [B, S, ...]`` (and ``w``) per table row ``[R, M]``
    (-1 = empty): fp32 sum in listed order, divided by the count, rounded once to the input
    dtype (``F.avg_pool2d``); ``round_sum``: the sum is rounded to the dtype first and the
    division rounded again (``gathered.sum(dim=2) / denom`` in the 16-bit dtype, :3976-3983)."""
    stf = torch.from_numpy(np.asarray(table))
    valid = stf >= 0
    cnt = valid.sum(-1).clamp(min=1).to(torch.float32)
    idx = stf.clamp(min=0).long()
    kf = k.float()
    acc = torch.zeros(k.shape[0], stf.shape[0], *k.shape[2:], dtype=torch.float32)
    for m in range(stf.shape[1]):
        vm = valid[:, m].to(torch.float32).view(1, -1, *([1] * (k.dim() - 2)))
        acc += kf[:, idx[:, m]] * vm
    if round_sum:
        acc = acc.to(k.dtype).float()
    out_k = (acc / cnt.view(1, -1, *([1] * (k.dim() - 2)))).to(k.dtype)
    if w is None:
        return out_k, None
    wf = w.float()
    accw = torch.zeros(w.shape[0], stf.shape[0], w.shape[2], dtype=torch.float32)
    for m in range(stf.shape[1]):
        accw += wf[:, idx[:, m]] * valid[:, m].to(torch.float32).view(1, -1, 1)
    if round_sum:
        accw = accw.to(w.dtype).float()
    return out_k, (accw / cnt.view(1, -1, 1)).to(w.dtype)


def static_pack4_table(sub_w: torch.Tensor, layout: Dict, sub: np.ndarray) -> np.ndarray:
    """Per batch element, the one sub-cell each coarse row expands to: the sub-cell whose
    gate, averaged over heads (fp32 sum times 1 / Hi, rounded to the dtype), is largest,
    the first on ties; special and edge rows keep their token. ``sub_w [B, C, 4, Hi]``;
    returns int64 ``[B, L, 4]`` (reference: dsa_attention.py:3521-3542)."""
    B, C, G, Hi = sub_w.shape
    L = int(layout["source_len"])
    off = int(layout["special_count"]) + int(layout["edge_count"])
    W = sub.shape[2]
    table = np.full((B, L, W), -1, dtype=np.int64)
    table[:, :off, 0] = layout["source_to_fine"][:off, 0]
    score = (sub_w.float().sum(-1) * (1.0 / Hi)).to(sub_w.dtype).float()  # [B, C, G]
    best = score.argmax(-1).numpy()  # first maximal index
    table[:, off:off + C] = sub[np.arange(C)[None, :], best]
    return table


def candidate_scores(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, rows: torch.Tensor,
                     softmax_scale: float) -> torch.Tensor:
    """fp32 indexer score of query t against key row rows[b, t, c] (-inf where < 0):
    sum_h w * relu(scale * <q, k>) (the formula of ``oracle.indexer.indexer_scores``)."""
    B, T, C = rows.shape
    safe = rows.clamp(min=0).long()
    qf, kf, wf = q.float(), k.float(), w.float()
    out = torch.empty(B, T, C, dtype=torch.float32)
    for b in range(B):
        kr = kf[b][safe[b]]  # [T, C, Hi, Di]
        z = torch.einsum("thd,tchd->tch", qf[b], kr) * torch.tensor(float(softmax_scale), dtype=torch.float32)
        out[b] = (torch.relu(z) * wf[b][safe[b]]).sum(-1, dtype=torch.float32)
    return torch.where(rows >= 0, out, torch.full_like(out, float("-inf")))


def rerank(q, k, w, coarse_indices: torch.Tensor, layout: Dict, topk: int, softmax_scale: float):
    """exact_rerank for given source rows ``[B, T, Kc]`` (reference: dsa_attention.py:
    3599-3635): the fine tokens of the chosen rows, in (row, slot) order, scored exactly;
    the top ``min(topk, fine_len)`` of them. Returns (tokens [B, T, target] int64,
    candidates [B, T, Kc * M], candidate scores) or None when a query has fewer valid
    candidates than the target (the caller then grows the coarse budget)."""
    stf = torch.from_numpy(layout["source_to_fine"])
    B, T, Kc = coarse_indices.shape
    fine_len = int(layout["tokens_per_view"]) * int(layout["num_views"])
    target = min(int(topk), fine_len)
    cand = stf[coarse_indices.reshape(-1).long()].reshape(B, T, -1)
    if bool(((cand >= 0).sum(-1) < target).any()):
        return None
    sc = candidate_scores(q, k, w, cand, softmax_scale)
    pick = sc.topk(target, dim=-1, sorted=False)[1]
    return cand.gather(-1, pick), cand, sc


def subcell_top1(q, sub_k, sub_w, ordered_rows: torch.Tensor, layout: Dict, sub: np.ndarray, topk: int,
                 softmax_scale: float):
    """subcell_top1 for chosen source rows in their expansion order (reference:
    dsa_attention.py:3629-3812). Every chosen special/edge row gives its token; the
    remaining budget ``ceil((target - singles) / 4)`` (at most the chosen cells' sub-cell
    count) goes to the best-scoring 2 x 2 sub-cells of the chosen cells (exact scores
    against the pooled sub-cell keys ``sub_k [B, C, 4, Hi, Di]``; ties: earlier position
    first). Output: the singles in row order, then the kept sub-cells' tokens in position
    order (row order, then sub-cell), cut to the target. Returns (tokens, sub-cell scores
    [B, T, Kc, 4] (-inf for special/edge rows), kept positions) or None when a query ends
    with fewer tokens than the target."""
    stf = layout["source_to_fine"]
    off = int(layout["special_count"]) + int(layout["edge_count"])
    B, T, Kc = ordered_rows.shape
    G, W = sub.shape[1], sub.shape[2]
    fine_len = int(layout["tokens_per_view"]) * int(layout["num_views"])
    target = min(int(topk), fine_len)
    rows = ordered_rows.long()
    cell = (rows - off).clamp(min=0)
    # sub-cell scores of every chosen row (special/edge rows masked to -inf)
    srow = torch.where((rows >= off).unsqueeze(-1), cell.unsqueeze(-1) * G + torch.arange(G), torch.tensor(-1))
    sk = sub_k.reshape(B, -1, *sub_k.shape[3:])
    sw = sub_w.reshape(B, -1, sub_w.shape[-1])
    scores = candidate_scores(q, sk, sw, srow.reshape(B, T, Kc * G), softmax_scale).reshape(B, T, Kc, G)
    out = torch.empty(B, T, target, dtype=torch.int64)
    kept_all = []
    for b in range(B):
        for t in range(T):
            singles = [int(stf[r, 0]) for r in rows[b, t].tolist() if r < off and stf[r, 0] >= 0]
            blocks = [(i, r) for i, r in enumerate(rows[b, t].tolist()) if r >= off]
            remain = max(target - len(singles), 0)
            keep = min((remain + W - 1) // W, len(blocks) * G)
            pos = [(i, g) for i, _ in blocks for g in range(G)]
            sc = [float(scores[b, t, i, g]) for i, g in pos]
            order = sorted(range(len(pos)), key=lambda j: (-sc[j], j))[:keep]
            kept = sorted(j for j in order if math.isfinite(sc[j]))
            toks = list(singles)
            for j in kept:
                i, g = pos[j]
                c = int(rows[b, t, i]) - off
                toks += [int(x) for x in sub[c, g] if x >= 0]
            if len(toks) < target:
                return None
            out[b, t] = torch.tensor(toks[:target])
            kept_all.append([pos[j] for j in kept])
    return out, scores, kept_all


def fine_to_source_row(layout: Dict) -> np.ndarray:
    """Source row of every fine token (-1 for none), reference: dsa_attention.py:3198-3208."""
    stf = layout["source_to_fine"]
    fine_len = int(layout["tokens_per_view"]) * int(layout["num_views"])
    f2r = np.full(fine_len, -1, dtype=np.int64)
    r, m = np.nonzero(stf >= 0)
    f2r[stf[r, m]] = r
    return f2r


def query_downsample(q: torch.Tensor, layout: Dict, q_offset: int):
    """(coarse queries [B, Nc, Hi, Di], fine_to_local [T]) for the query chunk q = queries
    q_offset .. q_offset + T (reference: dsa_attention.py:3929-3997): a source row all of
    whose tokens lie in the chunk becomes one query, the mean of its tokens' queries (sum
    rounded to the dtype, then divided by the count in the dtype); the tokens of the other
    rows stay single queries. Coarse queries: full rows by row index, then the single
    tokens in order."""
    T = q.shape[1]
    f2r = fine_to_source_row(layout)
    rows = f2r[q_offset:q_offset + T]
    if (rows < 0).any():
        raise RuntimeError("Invalid query downsample row mapping.")
    uniq, inv = np.unique(rows, return_inverse=True)
    counts = np.bincount(inv, minlength=uniq.size)
    full_counts = (layout["source_to_fine"] >= 0).sum(-1)[uniq]
    full = counts == full_counts
    tok_full = full[inv]
    stf = layout["source_to_fine"]
    table_full = np.where(stf[uniq[full]] >= 0, stf[uniq[full]] - q_offset, -1)
    partial = np.nonzero(~tok_full)[0]
    table = np.concatenate([table_full, np.full((partial.size, stf.shape[1]), -1, dtype=np.int64)], 0)
    table[table_full.shape[0]:, 0] = partial
    f2l = np.empty(T, dtype=np.int64)
    f2l[tok_full] = (np.cumsum(full) - 1)[inv[tok_full]]
    f2l[partial] = table_full.shape[0] + np.arange(partial.size)
    coarse_q, _ = pool_rows(q, None, table, round_sum=True)
    return coarse_q, f2l


def select_strategy(q, k, w, layout: Dict, topk: int, softmax_scale: float, strategy: str,
                    coarse_ratio: float = 1.1, pad_window: int = 64, recall_growth: float = 1.5,
                    recall_max_steps: int = 3, q_offset: int = 0, explicit_coarse: int = 0) -> torch.Tensor:
    """One query chunk through a resolved strategy (reference: dsa_attention.py:4187-4260),
    coarse top-k from the oracle scores, chosen rows expanded in ``order_by_score`` order.
    Returns fine token indices [B, T, target] (sets for exact_rerank)."""
    fine_len = int(layout["tokens_per_view"]) * int(layout["num_views"])
    target = min(int(topk), fine_len)
    L = int(layout["source_len"])
    kc = coarse_topk_for(layout, topk, strategy, coarse_ratio, explicit_coarse)

    def coarse(qq, sk, sw, n):
        sc = oidx.indexer_scores(qq, sk, sw, None, softmax_scale)
        v, i = sc.topk(min(n, sc.shape[-1]), dim=-1)
        return order_by_score(i, v)

    def full_indexer():
        sc = oidx.indexer_scores(q, k, w, None, softmax_scale)
        return sc.topk(target, dim=-1)[1]

    sk, sw = pool_sources(k, w, layout)
    if strategy == "legacy":
        return expand(coarse(q, sk, sw, kc), layout, topk, fine_len, pad_window)
    if strategy == "qk_sym_x2_broadcast":
        cq, f2l = query_downsample(q, layout, q_offset)
        fine = expand(coarse(cq, sk, sw, kc), layout, topk, fine_len, pad_window)
        return fine[:, torch.from_numpy(f2l)]
    sub = subcell_table(layout)
    if strategy == "subcell_static_pack4":
        if sub is None:
            return full_indexer()
        _, sub_w = pool_rows(k, w, sub.reshape(-1, sub.shape[2]))
        table = static_pack4_table(sub_w.reshape(k.shape[0], -1, sub.shape[1], w.shape[2]), layout, sub)
        lay = dict(layout, source_to_fine=None)
        rows = coarse(q, sk, sw, kc)
        out = []
        for b in range(q.shape[0]):
            lay["source_to_fine"] = table[b]
            out.append(expand(rows[b:b + 1], dict(lay, expand_round_robin=True), topk, fine_len, pad_window))
        return torch.cat(out, 0)
    attempt = min(max(kc, 1), L)
    sub_k = sub_w = None
    if strategy == "subcell_top1" and sub is not None:
        sub_k, sub_w = pool_rows(k, w, sub.reshape(-1, sub.shape[2]))
        sub_k = sub_k.reshape(k.shape[0], -1, sub.shape[1], *k.shape[2:])
        sub_w = sub_w.reshape(k.shape[0], -1, sub.shape[1], w.shape[2])
    for _ in range(max(int(recall_max_steps), 1)):
        rows = coarse(q, sk, sw, attempt)
        if strategy == "exact_rerank":
            got = rerank(q, k, w, rows, layout, topk, softmax_scale)
        else:
            got = None if sub is None else subcell_top1(q, sub_k, sub_w, rows, layout, sub, topk, softmax_scale)
        if got is not None:
            return got[0]
        if attempt >= L:
            break
        attempt = min(max(int(math.ceil(attempt * max(float(recall_growth), 1.1))), attempt + 1), L)
    return full_indexer()
