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
