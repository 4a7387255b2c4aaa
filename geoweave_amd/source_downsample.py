"""Source-downsample coarse selector on gfx950 (inference only, off unless requested).

An approximate top-k for many views: the indexer keys of each view's patch grid are
averaged over ``factor x factor`` cells, the indexer selects the top ``coarse_topk`` of
these source rows (special tokens and the edge tokens outside the pooled area are source
rows of their own), and each chosen row is expanded back to the fine tokens it covers.
With factor 2 at S = 32 views the indexer scores 43,968 x 12,864 pairs instead of
43,968^2. ``DSAAttention``'s selector (``easyvolcap/official_vggt/layers/dsa_attention.py``):
layout ``:3069-3259``, pooling ``:3386-3542``, coarse budget ``:3328-3375``, expansion
``:4079-4186``, dispatch ``:4187-4260,4279-4318``; defaults ``:122-132``.

Strategies (``:3273-3288``: ``qk_sym_x2_broadcast`` needs factor 2, the others factor >= 4,
anything else is "legacy"):

* ``legacy``: the chosen rows expand to all their tokens (round robin over the rows).
* ``exact_rerank`` (``:3599-3635``): the chosen rows' tokens are scored exactly and the top
  target kept (``gw_source_downsample_rerank``).
* ``subcell_top1`` (``:3629-3812``, factor 4): chosen special/edge rows give their token,
  the rest of the budget goes to the best 2 x 2 sub-cells of the chosen cells, scored
  against 2 x 2 pooled keys (``gw_source_downsample_subcell_top1``).
* ``subcell_static_pack4`` (``:3521-3542``, factor 4): each cell expands to one sub-cell,
  chosen per batch element by its pooled gates (``gw_source_downsample_static_pack4``),
  then the legacy expansion over that table.
* ``qk_sym_x2_broadcast`` (``:3929-4078``, factor 2): the queries are downsampled too (the
  mean of a cell's queries when the chunk holds the whole cell), one selection per coarse
  query, broadcast to its fine queries.

exact_rerank and subcell_top1 retry a query chunk with a coarse budget grown by
``recall_growth`` when a query runs short of candidates, up to ``recall_max_steps`` times,
then take the full indexer (``:4236-4260``); so do the sub-cell strategies when the layout
has no sub-cell keys (representative points). The reference computes the sub-cell keys only
for factor 4 (its reshape fails for larger factors); here the sub-cell strategies accept
factor 4 and raise otherwise.

Device steps: ``gw_source_downsample_pool`` (pooled keys and gates, pooled queries), the
indexer top-k (``gw_indexer_topk_fwd`` over the source rows) and the strategy's kernels
above. The layout tables are built once per shape on the host and cached on the device.

The reference only takes this path without a mask, without scores and outside training
(``:3044-3067``); the same preconditions hold here.

Order of the chosen source rows: the expansion is order dependent (round robin, then a
cut to top-k), and the reference takes the order of an unsorted ``torch.topk``
(``indexer.py:600-603``), which no API fixes. Here the rows are taken by score
descending, row index ascending on ties, so the result is reproducible, and the tokens cut
are those of the lowest-scoring rows. Candidate and sub-cell scores are the indexer's fp32
formula; the reference ranks them after rounding to the 16-bit dtype, with an unsorted
``torch.topk`` on ties. subcell_top1 keeps the best ``keep`` sub-cells of each query (the
reference keeps the first ``keep`` of an unsorted top ``max(keep)`` over the chunk) and lists
them in (row, sub-cell) order.
"""
from __future__ import annotations

import math
import threading
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _lib
from .custom_indexer.sparse_topk_indexer import sparse_topk_indexer_inference_func

__all__ = ["SourceDownsample", "SourceLayout", "build_layout", "select_topk"]

STRATEGIES = ("legacy", "exact_rerank", "subcell_top1", "subcell_static_pack4", "qk_sym_x2_broadcast")


@dataclass(frozen=True)
class SourceDownsample:
    """Selector settings (reference indexer config keys ``source_downsample_*``,
    ``dsa_attention.py:122-132``) plus the token layout of the call (the reference's
    ``state.tokens_per_view``, ``num_views``, ``patch_start_idx``, ``patch_grid_*``)."""

    tokens_per_view: int
    num_views: int
    patch_start_idx: int
    factor: int = 2
    coarse_topk: int = 0
    coarse_ratio: float = 1.1
    pad_window: int = 64
    representative_points: bool = False
    strategy: str = "legacy"
    grid_h: int = 0
    grid_w: int = 0
    recall_growth: float = 1.5      # source_downsample_recall_growth (:3298-3306)
    recall_max_steps: int = 3       # source_downsample_recall_max_steps (:3308-3316)
    query_chunk: int = 4096         # source_downsample_query_chunk (:3261-3271)


@dataclass
class SourceLayout:
    """Source rows of one (views, grid, factor) shape."""

    source_to_fine: np.ndarray  # int32 [L, M], -1 past a row's count
    special_count: int
    edge_count: int
    coarse_count: int
    round_robin: bool
    fine_len: int
    factor: int = 1
    # factor 4 without representative points: the tokens of each cell's 2 x 2 sub-cells,
    # int32 [coarse_count * 4, 4], sub-cell g = 2 sy + sx in (dy, dx) order (:3229-3257)
    subcell_to_fine: Optional[np.ndarray] = None

    @property
    def first_cell_row(self) -> int:
        return self.special_count + self.edge_count

    @property
    def source_len(self) -> int:
        return int(self.source_to_fine.shape[0])

    @property
    def max_block_tokens(self) -> int:
        return int(self.source_to_fine.shape[1])

    @property
    def mapped_tokens(self) -> int:
        return self.special_count + self.edge_count + self.coarse_count * self.max_block_tokens


def _patch_grid(image_tokens: int, grid_h: int, grid_w: int) -> Tuple[int, int]:
    # reference: dsa_attention.py:3034-3042 (explicit grid if consistent, else a square)
    if grid_h > 0 and grid_w > 0 and grid_h * grid_w == image_tokens:
        return grid_h, grid_w
    side = math.isqrt(max(image_tokens, 0))
    return (side, side) if side > 0 and side * side == image_tokens else (0, 0)


def build_layout(cfg: SourceDownsample) -> Optional[SourceLayout]:
    """Source rows in the reference's order (dsa_attention.py:3069-3259): the special tokens
    of all views, then each view's edge tokens (row-major, outside the pooled area), then
    each view's coarse cells (row-major), each cell listing its tokens in (dy, dx) order
    (or its representative points when ``factor > 2`` and ``representative_points``).
    None when the shape does not describe square-gridded views (the reference then uses
    the full indexer)."""
    f = max(int(cfg.factor), 1)
    tpv, nv, psi = int(cfg.tokens_per_view), int(cfg.num_views), int(cfg.patch_start_idx)
    if tpv <= 0 or nv <= 0 or psi < 0 or psi >= tpv:
        return None
    gh, gw = _patch_grid(tpv - psi, int(cfg.grid_h), int(cfg.grid_w))
    if gh <= 0 or gw <= 0:
        return None
    if f > 2 and cfg.representative_points:
        qt = max(f // 4, 0)
        lo, hi = min(qt, f - 1), max(min(f - 1 - qt, f - 1), 0)
        offs = list(dict.fromkeys([(lo, lo), (lo, hi), (hi, lo), (hi, hi)]))
        round_robin = False
    else:
        offs = [(dy, dx) for dy in range(f) for dx in range(f)]
        round_robin = True
    M = len(offs)
    ph, pw = gh // f * f, gw // f * f
    view0 = np.arange(nv, dtype=np.int64) * tpv
    special = (view0[:, None] + np.arange(psi)[None, :]).reshape(-1)
    ys, xs = np.meshgrid(np.arange(gh), np.arange(gw), indexing="ij")
    outside = ~((ys < ph) & (xs < pw))
    edge = (view0[:, None] + psi + (ys * gw + xs)[outside][None, :]).reshape(-1)
    cy, cx = np.meshgrid(np.arange(ph // f), np.arange(pw // f), indexing="ij")
    oy = np.array([o[0] for o in offs])
    ox = np.array([o[1] for o in offs])
    y = cy.reshape(-1, 1) * f + oy[None, :]
    x = cx.reshape(-1, 1) * f + ox[None, :]
    cell = np.where((y < gh) & (x < gw), y * gw + x, -1)  # [cells per view, M]
    coarse = np.where(cell[None] >= 0, view0[:, None, None] + psi + cell[None], -1).reshape(-1, M)
    single = np.full((special.size + edge.size, M), -1, dtype=np.int64)
    single[:, 0] = np.concatenate([special, edge])
    stf = np.concatenate([single, coarse], axis=0).astype(np.int32)
    sub = None
    if f == 4 and round_robin and coarse.shape[0] > 0:
        # sub-cell g takes the cell offsets (dy, dx) with (dy // 2, dx // 2) = divmod(g, 2)
        groups = [[dy * 4 + dx for dy in range(4) for dx in range(4) if (dy // 2) * 2 + dx // 2 == g]
                  for g in range(4)]
        sub = np.ascontiguousarray(np.stack([coarse[:, pos] for pos in groups], axis=1).reshape(-1, 4),
                                   dtype=np.int32)
    return SourceLayout(stf, int(special.size), int(edge.size), int(coarse.shape[0]), round_robin, tpv * nv, f, sub)


def resolve_strategy(strategy: Optional[str], factor: int) -> str:
    """The strategy a call runs (dsa_attention.py:3273-3288): qk_sym_x2_broadcast only at
    factor 2, the others only at factor >= 4; anything else is "legacy"."""
    st = str(strategy or "legacy").strip().lower()
    f = int(factor)
    if st == "qk_sym_x2_broadcast":
        return st if f == 2 else "legacy"
    if f < 4 and st != "legacy":
        return "legacy"
    return st if st in STRATEGIES else "legacy"


def coarse_budget(layout: SourceLayout, topk: int, cfg: SourceDownsample, strategy: Optional[str] = None) -> int:
    """Source rows to select (dsa_attention.py:3328-3375): topk over the average expansion
    (4 tokens per cell for the sub-cell strategies, :3290-3296), times coarse_ratio; if that
    would not even cover the special tokens, the specials plus the remaining budget over
    the non-special expansion. subcell_static_pack4: the specials plus the rest over 4."""
    L = layout.source_len
    if int(cfg.coarse_topk or 0) > 0:
        return min(max(int(cfg.coarse_topk), 1), L)
    st = strategy if strategy is not None else resolve_strategy(cfg.strategy, layout.factor)
    ratio = max(float(cfg.coarse_ratio or 1.1), 1.0)
    special = min(layout.special_count, int(topk))
    sub_expand = max(layout.factor // 2, 1) ** 2
    if st == "subcell_static_pack4":
        ct = special + math.ceil(float(max(int(topk) - special, 0)) / float(sub_expand) * ratio)
        return min(max(int(ct), 1), L)
    mapped = layout.mapped_tokens
    if st == "subcell_top1":
        mapped = layout.special_count + layout.edge_count + layout.coarse_count * sub_expand
    ct = math.ceil(float(topk) / max(mapped / L, 1.0) * ratio)
    ns_len = L - layout.special_count
    if 0 < special < int(topk) and ct < special and ns_len > 0:
        ns_avg = max((layout.mapped_tokens - layout.special_count) / ns_len, 1.0)
        if st == "subcell_top1":
            ns_avg = max(ns_avg / (layout.factor / 2.0) ** 2, 1.0)
        ct = max(ct, special + max(math.ceil(float(int(topk) - special) / ns_avg * ratio), 1))
    return min(max(int(ct), 1), L)


_cache_lock = threading.Lock()
_device_tables: Dict[Tuple, Tuple[SourceLayout, torch.Tensor, Optional[torch.Tensor]]] = {}
_query_plans: Dict[Tuple, Tuple[torch.Tensor, torch.Tensor]] = {}


def _layout_key(cfg: SourceDownsample) -> Tuple:
    return (cfg.tokens_per_view, cfg.num_views, cfg.patch_start_idx, cfg.factor, cfg.grid_h, cfg.grid_w,
            bool(cfg.representative_points))


def _layout_on(cfg: SourceDownsample, device: torch.device):
    """(layout, device source_to_fine, device sub-cell table or None), cached per shape."""
    key = _layout_key(cfg) + (device,)
    with _cache_lock:
        hit = _device_tables.get(key)
    if hit is not None:
        return hit
    layout = build_layout(cfg)
    if layout is None:
        return None
    sub = None if layout.subcell_to_fine is None else torch.from_numpy(layout.subcell_to_fine).to(device)
    entry = (layout, torch.from_numpy(layout.source_to_fine).to(device), sub)
    with _cache_lock:
        _device_tables[key] = entry
    return entry


def pool_rows(x: torch.Tensor, g: Optional[torch.Tensor], table: torch.Tensor,
              round_sum: bool = False) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """The mean of the rows of ``x [B, S, Hi, Di]`` (and gates ``g [B, S, Hi]``) each table
    row ``[R, M]`` lists (-1 = none), via gw_source_downsample_pool: fp32 sum / count,
    rounded once (or, ``round_sum``, the sum rounded before the division)."""
    x = x.contiguous()
    table = table.contiguous()
    B, S, Hi, Di = x.shape
    R, M = table.shape
    ox = torch.empty(B, R, Hi, Di, device=x.device, dtype=x.dtype)
    og = None
    if g is not None:
        g = g.to(x.dtype).contiguous()
        og = torch.empty(B, R, Hi, device=x.device, dtype=x.dtype)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_pool(_lib.dtype_code(x.dtype), x.data_ptr(), _lib.ptr(g), B, S, Hi, Di,
                                             table.data_ptr(), R, M, int(bool(round_sum)), ox.data_ptr(),
                                             _lib.ptr(og), _lib.stream_handle(x.device)),
               "gw_source_downsample_pool")
    return ox, og


def pool_sources(k: torch.Tensor, w: torch.Tensor, table: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(source_k [B, L, Hi, Di], source_w [B, L, Hi]) via gw_source_downsample_pool."""
    return pool_rows(k, w, table)


def expand(coarse_idx: torch.Tensor, layout: SourceLayout, table: torch.Tensor, target: int,
           pad_window: int, coarse_scores: Optional[torch.Tensor] = None, row_map: Optional[torch.Tensor] = None,
           round_robin: Optional[bool] = None) -> torch.Tensor:
    """int32 fine indices [B, T, target] via gw_source_downsample_expand; with
    ``coarse_scores`` the chosen rows are taken by score descending (row ascending on
    ties), else in their given order. ``table``: ``[L, M]``, or ``[B, L, M]`` per batch
    element. ``row_map`` (int32 [T_out]): output row t expands chosen row ``row_map[t]``."""
    coarse_idx = coarse_idx.to(torch.int32).contiguous()
    B, T, Kc = coarse_idx.shape
    dtype = torch.bfloat16
    if coarse_scores is not None:
        if coarse_scores.dtype not in (torch.bfloat16, torch.float16) or coarse_scores.shape != coarse_idx.shape:
            raise ValueError("coarse_scores must be bf16/fp16 with the shape of coarse_idx")
        coarse_scores = coarse_scores.contiguous()
        dtype = coarse_scores.dtype
    if table.dim() == 3:
        if table.shape[0] != B:
            raise ValueError("a per-batch table needs one [L, M] table per batch element")
        L, M = table.shape[1], table.shape[2]
        tsb = L * M
    else:
        L, M = table.shape
        tsb = 0
    table = table.contiguous()
    t_out = T
    if row_map is not None:
        row_map = row_map.to(device=coarse_idx.device, dtype=torch.int32).contiguous()
        t_out = row_map.shape[0]
    rr = layout.round_robin if round_robin is None else bool(round_robin)
    out = torch.empty(B, t_out, target, device=coarse_idx.device, dtype=torch.int32)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_expand(
        _lib.dtype_code(dtype), coarse_idx.data_ptr(), _lib.ptr(coarse_scores),
        coarse_idx.stride(0), coarse_idx.stride(1), B, T, Kc, table.data_ptr(), tsb,
        L, M, int(rr), target, max(1, min(int(pad_window or 64), target)), _lib.ptr(row_map), t_out,
        out.data_ptr(), _lib.stream_handle(coarse_idx.device)),
        "gw_source_downsample_expand")
    return out


def rerank(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, coarse_idx: torch.Tensor, layout: SourceLayout,
           table: torch.Tensor, target: int, softmax_scale: float) -> Tuple[torch.Tensor, bool]:
    """exact_rerank of given chosen rows ``coarse_idx [B, T, Kc]`` via
    gw_source_downsample_rerank: (int32 [B, T, target], every query had enough
    candidates). The out rows are unspecified when the flag is False."""
    q = q.contiguous()
    k = k.contiguous()
    w = w.to(k.dtype).contiguous()
    coarse_idx = coarse_idx.to(torch.int32).contiguous()
    table = table.contiguous()
    B, T, Hi, Di = q.shape
    Kc = coarse_idx.shape[-1]
    out = torch.empty(B, T, target, device=q.device, dtype=torch.int32)
    fail = torch.zeros(1, device=q.device, dtype=torch.int32)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_rerank(
        _lib.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), w.data_ptr(), B, T, k.shape[1], Hi, Di,
        coarse_idx.data_ptr(), coarse_idx.stride(0), coarse_idx.stride(1), Kc, table.data_ptr(),
        layout.source_len, layout.max_block_tokens, target, float(softmax_scale), out.data_ptr(), fail.data_ptr(),
        _lib.stream_handle(q.device)), "gw_source_downsample_rerank")
    return out, not bool(fail.item())


def subcell_top1(q: torch.Tensor, sub_k: torch.Tensor, sub_w: torch.Tensor, coarse_idx: torch.Tensor,
                 coarse_scores: torch.Tensor, layout: SourceLayout, table: torch.Tensor, sub_table: torch.Tensor,
                 target: int, softmax_scale: float) -> Tuple[torch.Tensor, bool]:
    """subcell_top1 of given chosen rows (expanded by score descending) via
    gw_source_downsample_subcell_top1; ``sub_k [B, C * 4, Hi, Di]`` / ``sub_w`` are the
    pooled sub-cell keys and gates. (int32 [B, T, target], every query had enough tokens)."""
    q = q.contiguous()
    coarse_idx = coarse_idx.to(torch.int32).contiguous()
    coarse_scores = coarse_scores.contiguous()
    table, sub_table = table.contiguous(), sub_table.contiguous()
    sub_k, sub_w = sub_k.contiguous(), sub_w.to(sub_k.dtype).contiguous()
    B, T, Hi, Di = q.shape
    Kc = coarse_idx.shape[-1]
    C = layout.coarse_count
    G, W = 4, sub_table.shape[1]
    out = torch.empty(B, T, target, device=q.device, dtype=torch.int32)
    fail = torch.zeros(1, device=q.device, dtype=torch.int32)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_subcell_top1(
        _lib.dtype_code(q.dtype), q.data_ptr(), sub_k.data_ptr(), sub_w.data_ptr(), B, T, C, G, Hi, Di,
        coarse_idx.data_ptr(), coarse_scores.data_ptr(), coarse_idx.stride(0), coarse_idx.stride(1), Kc,
        table.data_ptr(), layout.source_len, layout.max_block_tokens, layout.first_cell_row, sub_table.data_ptr(),
        W, target, float(softmax_scale), out.data_ptr(), fail.data_ptr(), _lib.stream_handle(q.device)),
        "gw_source_downsample_subcell_top1")
    return out, not bool(fail.item())


def static_pack4_table(sub_w: torch.Tensor, layout: SourceLayout, table: torch.Tensor,
                       sub_table: torch.Tensor) -> torch.Tensor:
    """int32 [B, L, 4]: the one sub-cell each cell expands to under subcell_static_pack4
    (gw_source_downsample_static_pack4); special and edge rows keep their token."""
    B = sub_w.shape[0]
    table, sub_table = table.contiguous(), sub_table.contiguous()
    W = sub_table.shape[1]
    out = torch.empty(B, layout.source_len, W, device=sub_w.device, dtype=torch.int32)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_static_pack4(
        _lib.dtype_code(sub_w.dtype), sub_w.contiguous().data_ptr(), B, layout.coarse_count, 4, sub_w.shape[-1],
        table.data_ptr(), layout.source_len, layout.max_block_tokens, layout.first_cell_row, sub_table.data_ptr(),
        W, out.data_ptr(), _lib.stream_handle(sub_w.device)), "gw_source_downsample_static_pack4")
    return out


def _query_plan(cfg: SourceDownsample, layout: SourceLayout, q_offset: int, n: int, device: torch.device):
    """(pooling table [Nc, M], fine_to_local [n]) of the query chunk q_offset .. q_offset + n
    (dsa_attention.py:3929-3997): a source row all of whose tokens are in the chunk becomes
    one coarse query (its tokens' mean), the tokens of the other rows stay single queries;
    full rows by row index, then the single tokens in order."""
    key = _layout_key(cfg) + (int(q_offset), int(n), device)
    with _cache_lock:
        hit = _query_plans.get(key)
    if hit is not None:
        return hit
    stf = layout.source_to_fine.astype(np.int64)
    f2r = np.full(layout.fine_len, -1, dtype=np.int64)
    r, m = np.nonzero(stf >= 0)
    f2r[stf[r, m]] = r
    if q_offset < 0 or q_offset + n > layout.fine_len:
        raise ValueError(f"query chunk {q_offset}..{q_offset + n} outside the {layout.fine_len} layout tokens")
    rows = f2r[q_offset:q_offset + n]
    if (rows < 0).any():
        raise RuntimeError("Invalid query downsample row mapping.")
    uniq, inv = np.unique(rows, return_inverse=True)
    counts = np.bincount(inv, minlength=uniq.size)
    full = counts == (stf >= 0).sum(-1)[uniq]
    tok_full = full[inv]
    table_full = np.where(stf[uniq[full]] >= 0, stf[uniq[full]] - q_offset, -1)
    partial = np.nonzero(~tok_full)[0]
    table = np.concatenate([table_full, np.full((partial.size, stf.shape[1]), -1, dtype=np.int64)], 0)
    table[table_full.shape[0]:, 0] = partial
    f2l = np.empty(n, dtype=np.int64)
    f2l[tok_full] = (np.cumsum(full) - 1)[inv[tok_full]]
    f2l[partial] = table_full.shape[0] + np.arange(partial.size)
    entry = (torch.from_numpy(table.astype(np.int32)).to(device), torch.from_numpy(f2l.astype(np.int32)).to(device))
    with _cache_lock:
        _query_plans[key] = entry
    return entry


def query_downsample(q: torch.Tensor, cfg: SourceDownsample, q_offset: int = 0):
    """(coarse queries [B, Nc, Hi, Di], fine_to_local int32 [T]) of the query chunk ``q``
    starting at token ``q_offset`` (qk_sym_x2_broadcast, dsa_attention.py:3929-3997): the
    mean of a full row's queries is the dtype sum divided by the count in the dtype."""
    entry = _layout_on(cfg, q.device)
    if entry is None:
        raise ValueError("the source-downsample layout does not apply to this shape")
    layout = entry[0]
    table, f2l = _query_plan(cfg, layout, int(q_offset), q.shape[1], q.device)
    cq, _ = pool_rows(q, None, table, round_sum=True)
    return cq, f2l


@dataclass
class Prepared:
    """Pooled source keys of one call (and the strategy's extra tables)."""

    layout: SourceLayout
    table: torch.Tensor                     # int32 [L, M]
    source_k: torch.Tensor                  # [B, L, Hi, Di]
    source_w: torch.Tensor                  # [B, L, Hi]
    strategy: str
    sub_table: Optional[torch.Tensor] = None     # int32 [C * 4, 4]
    sub_k: Optional[torch.Tensor] = None         # [B, C * 4, Hi, Di] (subcell_top1)
    sub_w: Optional[torch.Tensor] = None         # [B, C * 4, Hi]
    static_table: Optional[torch.Tensor] = None  # int32 [B, L, 4] (subcell_static_pack4)


def prepare(k: torch.Tensor, w: torch.Tensor, cfg: SourceDownsample) -> Optional[Prepared]:
    """Pooled source keys (and the sub-cell keys or static table the strategy reads), or
    None if the layout does not apply (dsa_attention.py:3386-3542)."""
    entry = _layout_on(cfg, k.device)
    if entry is None or entry[0].fine_len != k.shape[1]:
        return None
    layout, table, sub = entry
    strategy = resolve_strategy(cfg.strategy, layout.factor)
    if strategy in ("subcell_top1", "subcell_static_pack4") and layout.factor != 4:
        raise ValueError(f"source-downsample strategy {strategy!r} needs factor 4 (the reference's 2 x 2 sub-cell "
                         f"keys exist only then), got factor {layout.factor}")
    sk, sw = pool_sources(k, w, table)
    prep = Prepared(layout, table, sk, sw, strategy, sub)
    if sub is not None and strategy == "subcell_top1":
        prep.sub_k, prep.sub_w = pool_rows(k, w, sub)
    elif sub is not None and strategy == "subcell_static_pack4":
        _, sub_w = pool_rows(k, w, sub)
        prep.static_table = static_pack4_table(sub_w, layout, table, sub)
    return prep


def _coarse(q, prep: Prepared, n: int, scale: float):
    empty = q.new_empty(0)
    return sparse_topk_indexer_inference_func(q, prep.source_k, prep.source_w, empty, int(n), float(scale), 256, 0)


def _select_chunk(q, k, w, prep: Prepared, cfg: SourceDownsample, topk: int, scale: float, q_offset: int):
    """One query chunk (dsa_attention.py:4187-4260)."""
    layout = prep.layout
    target = min(int(topk), layout.fine_len)
    kc = coarse_budget(layout, int(topk), cfg, prep.strategy)
    st = prep.strategy
    if st == "legacy":
        cidx, csc = _coarse(q, prep, kc, scale)
        return expand(cidx, layout, prep.table, target, cfg.pad_window, csc)
    if st == "qk_sym_x2_broadcast":
        cq, f2l = query_downsample(q, cfg, q_offset)
        cidx, csc = _coarse(cq, prep, kc, scale)
        return expand(cidx, layout, prep.table, target, cfg.pad_window, csc, row_map=f2l)
    if st == "subcell_static_pack4":
        if prep.static_table is None:
            return _full_indexer(q, k, w, topk, scale)
        cidx, csc = _coarse(q, prep, kc, scale)
        return expand(cidx, layout, prep.static_table, target, cfg.pad_window, csc, round_robin=True)
    if st == "subcell_top1" and prep.sub_k is None:
        return _full_indexer(q, k, w, topk, scale)  # no sub-cell keys: every attempt fails
    attempt = min(max(int(kc), 1), layout.source_len)
    growth = max(float(cfg.recall_growth or 1.5), 1.1)
    for _ in range(max(int(cfg.recall_max_steps or 3), 1)):
        cidx, csc = _coarse(q, prep, attempt, scale)
        if st == "exact_rerank":
            out, ok = rerank(q, k, w, cidx, layout, prep.table, target, scale)
        else:
            out, ok = subcell_top1(q, prep.sub_k, prep.sub_w, cidx, csc, layout, prep.table, prep.sub_table,
                                   target, scale)
        if ok:
            return out
        if attempt >= layout.source_len:
            break
        attempt = min(max(int(math.ceil(attempt * growth)), attempt + 1), layout.source_len)
    return _full_indexer(q, k, w, topk, scale)


def _full_indexer(q, k, w, topk, scale):
    idx, _ = sparse_topk_indexer_inference_func(q, k, w, q.new_empty(0), int(topk), float(scale), 256, 0)
    return idx


def select_topk(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, topk: int, softmax_scale: float,
                cfg: SourceDownsample, query_chunk: Optional[int] = None,
                prepared: Optional[Prepared] = None, q_offset: int = 0) -> Optional[torch.Tensor]:
    """Approximate top-k fine indices (int32 ``[B, T, min(topk, fine_len)]``) of the
    indexer queries ``q [B, T, Hi, Di]`` (tokens ``q_offset ..`` of the sequence) over the
    keys ``k [B, S, Hi, Di]`` / gates ``w [B, S, Hi]``, or None when the layout does not
    apply (S != tokens_per_view * num_views, or non-square grids): the caller then runs
    the full indexer, as the reference does (dsa_attention.py:4279-4318). Queries go in
    chunks of ``query_chunk`` (default ``cfg.query_chunk``), as the reference's do: the
    retries of exact_rerank / subcell_top1 and the query cells of qk_sym_x2_broadcast are
    per chunk (legacy and subcell_static_pack4 rows do not depend on the chunking and run
    in one pass unless ``query_chunk`` is given). ``prepared`` reuses ``prepare(...)``'s
    pooled keys across calls."""
    if int(cfg.factor) <= 1:
        return None
    prepared = prepared if prepared is not None else prepare(k, w, cfg)
    if prepared is None:
        return None
    T = q.shape[1]
    qc = int(query_chunk) if query_chunk else int(cfg.query_chunk or 0)
    if prepared.strategy in ("legacy", "subcell_static_pack4") and not query_chunk:
        qc = 0  # rows are independent of the chunking here: one pass
    step = T if qc <= 0 else min(qc, T)
    parts = []
    for s0 in range(0, T, max(step, 1)):
        parts.append(_select_chunk(q[:, s0:s0 + step].contiguous(), k, w, prepared, cfg, int(topk),
                                   float(softmax_scale), int(q_offset) + s0))
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)
