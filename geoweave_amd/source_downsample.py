"""Source-downsample coarse selector on gfx950 (inference only, off unless requested).

An approximate top-k for many views: the indexer keys of each view's patch grid are
averaged over ``factor x factor`` cells, the indexer selects the top ``coarse_topk`` of
these source rows (special tokens and the edge tokens outside the pooled area are source
rows of their own), and each chosen row is expanded back to the fine tokens it covers.
With factor 2 at S = 32 views the indexer scores 43,968 x 12,864 pairs instead of
43,968^2. This is the reference's "legacy" strategy of ``DSAAttention``
(``easyvolcap/official_vggt/layers/dsa_attention.py``): layout ``:3069-3259``, pooling
``:3386-3542``, coarse budget ``:3328-3375``, expansion ``:4079-4128``, dispatch
``:4187-4217,4279-4318``; defaults ``:122-132``.

Device steps: ``gw_source_downsample_pool`` (pooled keys and gates), the indexer top-k
(``gw_indexer_topk_fwd`` over the source rows) and ``gw_source_downsample_expand``. The
layout tables are built once per shape on the host and cached on the device.

Not implemented: the reference's other strategies (``exact_rerank``, ``subcell_top1``,
``subcell_static_pack4``, ``qk_sym_x2_broadcast``, ``:3599-4078``); asking for one raises.
The reference only takes this path without a mask, without scores and outside training
(``:3044-3067``); the same preconditions hold here.

Order of the chosen source rows: the expansion is order dependent (round robin, then a
cut to top-k), and the reference takes the order of an unsorted ``torch.topk``
(``indexer.py:600-603``), which no API fixes. Here the rows are taken by score
descending, row index ascending on ties, so the result is reproducible and does not
depend on query chunking, and the tokens cut are those of the lowest-scoring rows.
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

_STRATEGIES_NOT_BUILT = {"exact_rerank", "subcell_top1", "subcell_static_pack4", "qk_sym_x2_broadcast"}


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


@dataclass
class SourceLayout:
    """Source rows of one (views, grid, factor) shape."""

    source_to_fine: np.ndarray  # int32 [L, M], -1 past a row's count
    special_count: int
    edge_count: int
    coarse_count: int
    round_robin: bool
    fine_len: int

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
    return SourceLayout(stf, int(special.size), int(edge.size), int(coarse.shape[0]), round_robin, tpv * nv)


def coarse_budget(layout: SourceLayout, topk: int, cfg: SourceDownsample) -> int:
    """Source rows to select (dsa_attention.py:3328-3375, legacy strategy): topk over the
    average expansion, times coarse_ratio; if that would not even cover the special
    tokens, the specials plus the remaining budget over the non-special expansion."""
    L = layout.source_len
    if int(cfg.coarse_topk or 0) > 0:
        return min(max(int(cfg.coarse_topk), 1), L)
    ratio = max(float(cfg.coarse_ratio or 1.1), 1.0)
    ct = math.ceil(float(topk) / max(layout.mapped_tokens / L, 1.0) * ratio)
    special = min(layout.special_count, int(topk))
    ns_len = L - layout.special_count
    if 0 < special < int(topk) and ct < special and ns_len > 0:
        ns_avg = max((layout.mapped_tokens - layout.special_count) / ns_len, 1.0)
        ct = max(ct, special + max(math.ceil(float(int(topk) - special) / ns_avg * ratio), 1))
    return min(max(int(ct), 1), L)


_cache_lock = threading.Lock()
_device_tables: Dict[Tuple, Tuple[SourceLayout, torch.Tensor]] = {}


def _layout_on(cfg: SourceDownsample, device: torch.device) -> Optional[Tuple[SourceLayout, torch.Tensor]]:
    key = (cfg.tokens_per_view, cfg.num_views, cfg.patch_start_idx, cfg.factor, cfg.grid_h, cfg.grid_w,
           bool(cfg.representative_points), device)
    with _cache_lock:
        hit = _device_tables.get(key)
    if hit is not None:
        return hit
    layout = build_layout(cfg)
    if layout is None:
        return None
    entry = (layout, torch.from_numpy(layout.source_to_fine).to(device))
    with _cache_lock:
        _device_tables[key] = entry
    return entry


def pool_sources(k: torch.Tensor, w: torch.Tensor, table: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(source_k [B, L, Hi, Di], source_w [B, L, Hi]) via gw_source_downsample_pool."""
    k = k.contiguous()
    w = w.to(k.dtype).contiguous()
    B, S, Hi, Di = k.shape
    L, M = table.shape
    sk = torch.empty(B, L, Hi, Di, device=k.device, dtype=k.dtype)
    sw = torch.empty(B, L, Hi, device=k.device, dtype=k.dtype)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_pool(_lib.dtype_code(k.dtype), k.data_ptr(), w.data_ptr(), B, S, Hi, Di,
                                             table.data_ptr(), L, M, sk.data_ptr(), sw.data_ptr(),
                                             _lib.stream_handle(k.device)), "gw_source_downsample_pool")
    return sk, sw


def expand(coarse_idx: torch.Tensor, layout: SourceLayout, table: torch.Tensor, target: int,
           pad_window: int, coarse_scores: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int32 fine indices [B, T, target] via gw_source_downsample_expand; with
    ``coarse_scores`` the chosen rows are taken by score descending (row ascending on
    ties), else in their given order."""
    coarse_idx = coarse_idx.to(torch.int32).contiguous()
    B, T, Kc = coarse_idx.shape
    dtype = torch.bfloat16
    if coarse_scores is not None:
        if coarse_scores.dtype not in (torch.bfloat16, torch.float16) or coarse_scores.shape != coarse_idx.shape:
            raise ValueError("coarse_scores must be bf16/fp16 with the shape of coarse_idx")
        coarse_scores = coarse_scores.contiguous()
        dtype = coarse_scores.dtype
    out = torch.empty(B, T, target, device=coarse_idx.device, dtype=torch.int32)
    lib = _lib.load()
    _lib.check(lib.gw_source_downsample_expand(
        _lib.dtype_code(dtype), coarse_idx.data_ptr(), _lib.ptr(coarse_scores),
        coarse_idx.stride(0), coarse_idx.stride(1), B, T, Kc, table.data_ptr(),
        layout.source_len, layout.max_block_tokens, int(layout.round_robin), target,
        max(1, min(int(pad_window or 64), target)), out.data_ptr(), _lib.stream_handle(coarse_idx.device)),
        "gw_source_downsample_expand")
    return out


def select_topk(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, topk: int, softmax_scale: float,
                cfg: SourceDownsample, query_chunk: Optional[int] = None,
                prepared: Optional[Tuple] = None) -> Optional[torch.Tensor]:
    """Approximate top-k fine indices (int32 ``[B, T, min(topk, fine_len)]``) of the
    indexer queries ``q [B, T, Hi, Di]`` over the keys ``k [B, S, Hi, Di]`` / gates
    ``w [B, S, Hi]``, or None when the layout does not apply (S != tokens_per_view *
    num_views, or non-square grids): the caller then runs the full indexer, as the
    reference does (dsa_attention.py:4279-4318). ``prepared`` reuses ``prepare(...)``'s
    pooled keys across query chunks."""
    if cfg.strategy in _STRATEGIES_NOT_BUILT:
        raise NotImplementedError(f"source-downsample strategy {cfg.strategy!r} is not built (only 'legacy')")
    if int(cfg.factor) <= 1:
        return None
    prepared = prepared if prepared is not None else prepare(k, w, cfg)
    if prepared is None:
        return None
    layout, table, sk, sw = prepared
    target = min(int(topk), layout.fine_len)
    kc = coarse_budget(layout, int(topk), cfg)
    empty = q.new_empty(0)
    T = q.shape[1]
    step = T if not query_chunk or query_chunk <= 0 else min(int(query_chunk), T)
    parts = []
    for s0 in range(0, T, step):
        cidx, csc = sparse_topk_indexer_inference_func(q[:, s0:s0 + step], sk, sw, empty, kc, float(softmax_scale),
                                                       256, 0)
        parts.append(expand(cidx, layout, table, target, cfg.pad_window, csc))
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)


def prepare(k: torch.Tensor, w: torch.Tensor, cfg: SourceDownsample):
    """(layout, device table, source_k, source_w) or None if the layout does not apply."""
    entry = _layout_on(cfg, k.device)
    if entry is None or entry[0].fine_len != k.shape[1]:
        return None
    layout, table = entry
    sk, sw = pool_sources(k, w, table)
    return layout, table, sk, sw
