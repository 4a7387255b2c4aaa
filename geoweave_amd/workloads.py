"""Seeded synthetic inputs for one sparse global-attention layer.

Shapes follow a VGGT/Pi3 global-attention layer: B images-batches, S views of
P = 1374 tokens (37 x 37 patches at 518 px / patch 14, plus 5 special tokens), N = S * P
tokens, 16 attention heads of dim 64 (reference ``easyvolcap/official_vggt/models/
aggregator.py:66-68``), an indexer of 4 heads x 64 (``geoweave/configs/vggt.json:26,33``)
and top-k 1024 (``vggt.json:40``).

Recipe (all drawn on the CPU with a ``torch.Generator`` so the GPU and CPU sides see the
same values): x ~ N(0, 1) ``[B, N, 1024]``; indexer q = x Wq, k = x Wk with
Wq, Wk ~ N(0, 1/1024) ``[1024, 256]`` (about N(0, 1) per element); w = 1 + x Ww with
Ww ~ N(0, 0.25/1024) ``[1024, 4]`` (the gate's bias-1 init, ``indexer.py:63-68``, with a
spread that rarely crosses 0); attention q, k, v ~ N(0, 1). Seed = 20261201 + S, plus b
for batch element b. Values are rounded once to the compute dtype; the oracle upcasts the
same rounded values.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

TOKENS_PER_VIEW = 1374
DIM = 1024
ATTN_HEADS = 16
HEAD_DIM = 64
INDEXER_HEADS = 4
INDEXER_DIM = 64
TOPK = 1024
BASE_SEED = 20261201


@dataclass
class LayerInputs:
    q_idx: torch.Tensor   # [B, N, Hi, Di]
    k_idx: torch.Tensor   # [B, N, Hi, Di]
    w_idx: torch.Tensor   # [B, N, Hi]
    q: torch.Tensor       # [B, N, H, D]
    k: torch.Tensor       # [B, N, H, D]
    v: torch.Tensor       # [B, N, H, D]
    views: int
    batch: int

    @property
    def tokens(self) -> int:
        return int(self.q.shape[1])


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    return g


def indexer_inputs(
    views: int,
    batch: int = 1,
    dtype: torch.dtype = torch.bfloat16,
    tokens: Optional[int] = None,
    seed: Optional[int] = None,
):
    """(q, k, w) of the lightning indexer, CPU tensors in ``dtype``."""
    n = int(tokens) if tokens is not None else views * TOKENS_PER_VIEW
    base = BASE_SEED + views if seed is None else int(seed)
    qs, ks, ws = [], [], []
    for b in range(batch):
        g = _gen(base + b)
        wq = torch.randn(DIM, INDEXER_HEADS * INDEXER_DIM, generator=g) / DIM ** 0.5
        wk = torch.randn(DIM, INDEXER_HEADS * INDEXER_DIM, generator=g) / DIM ** 0.5
        ww = torch.randn(DIM, INDEXER_HEADS, generator=g) * (0.5 / DIM ** 0.5)
        x = torch.randn(n, DIM, generator=g)
        qs.append((x @ wq).view(n, INDEXER_HEADS, INDEXER_DIM))
        ks.append((x @ wk).view(n, INDEXER_HEADS, INDEXER_DIM))
        ws.append(1.0 + x @ ww)
    return (
        torch.stack(qs).to(dtype).contiguous(),
        torch.stack(ks).to(dtype).contiguous(),
        torch.stack(ws).to(dtype).contiguous(),
    )


def attention_inputs(
    views: int,
    batch: int = 1,
    dtype: torch.dtype = torch.bfloat16,
    tokens: Optional[int] = None,
    heads: int = ATTN_HEADS,
    head_dim: int = HEAD_DIM,
    seed: Optional[int] = None,
):
    """(q, k, v) of the attention, ``[B, N, H, D]`` CPU tensors in ``dtype``."""
    n = int(tokens) if tokens is not None else views * TOKENS_PER_VIEW
    base = BASE_SEED + views if seed is None else int(seed)
    out = []
    for b in range(batch):
        g = _gen(base + 7919 + b)
        out.append(torch.randn(3, n, heads, head_dim, generator=g))
    qkv = torch.stack(out, dim=1).to(dtype)
    return qkv[0].contiguous(), qkv[1].contiguous(), qkv[2].contiguous()


def random_positions(
    batch: int,
    tgt_len: int,
    src_len: int,
    topk: int,
    seed: int,
    invalid_fraction: float = 0.0,
) -> torch.Tensor:
    """int32 ``[B, T, K]`` distinct positions per row (random subsets of [0, S)), with an
    optional ragged tail of -1 entries like the reference test generator
    (``tests/sparse_index_flash_attn_tests.py:37-44``)."""
    g = _gen(seed)
    kk = min(topk, src_len)
    scores = torch.rand(batch, tgt_len, src_len, generator=g)
    pos = scores.topk(kk, dim=-1).indices.to(torch.int32)
    if invalid_fraction > 0:
        lengths = (kk * (1.0 - invalid_fraction * torch.rand(batch, tgt_len, generator=g))).long().clamp(min=1)
        ar = torch.arange(kk).view(1, 1, kk)
        pos = torch.where(ar < lengths.unsqueeze(-1), pos, torch.full_like(pos, -1))
    return pos.contiguous()


def distinct_positions(batch: int, tgt_len: int, src_len: int, topk: int, seed: int,
                       hub: Optional[int] = None) -> torch.Tensor:
    """int32 ``[B, T, K]`` positions with no repeat inside a row, cheap at any size: row t
    lists ``(off_t + j * step_t) mod S`` for j < K, with a random offset and a random step
    coprime to S (so the K entries are distinct when K <= S). ``hub``: key listed in every
    row that does not already list it (at j = 0), like a key the indexer picks for most
    queries."""
    import math

    g = _gen(seed)
    kk = min(topk, src_len)
    cands = [s for s in range(1, min(src_len, 4096)) if math.gcd(s, src_len) == 1] or [1]
    steps = torch.tensor(cands)[torch.randint(0, len(cands), (batch, tgt_len, 1), generator=g)]
    off = torch.randint(0, src_len, (batch, tgt_len, 1), generator=g)
    j = torch.arange(kk).view(1, 1, kk)
    pos = (off + j * steps) % src_len
    if hub is not None:
        free = ~(pos == hub).any(-1)
        pos[..., 0] = torch.where(free, torch.full_like(pos[..., 0], hub), pos[..., 0])
    return pos.to(torch.int32).contiguous()


def layer_inputs(views: int, batch: int = 1, dtype: torch.dtype = torch.bfloat16,
                 tokens: Optional[int] = None) -> LayerInputs:
    qi, ki, wi = indexer_inputs(views, batch, dtype, tokens)
    q, k, v = attention_inputs(views, batch, dtype, tokens)
    return LayerInputs(qi, ki, wi, q, k, v, views, batch)


PATCH_GRID = 37
SPECIAL_TOKENS = 5


def patch_positions(views: int, batch: int = 1) -> torch.Tensor:
    """int32 ``[B, S * P, 2]`` (y, x) rotary positions of the global-attention tokens: per
    view 5 special tokens at (0, 0), then the 37 x 37 patch grid at (row + 1, col + 1)
    (reference ``easyvolcap/official_vggt/models/aggregator.py:515-526``)."""
    ys, xs = torch.meshgrid(torch.arange(PATCH_GRID), torch.arange(PATCH_GRID), indexing="ij")
    grid = torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1
    one = torch.cat([torch.zeros(SPECIAL_TOKENS, 2, dtype=grid.dtype), grid], 0)
    return one.repeat(views, 1).unsqueeze(0).expand(batch, -1, -1).to(torch.int32).contiguous()


def layer_module_inputs(views: int, batch: int = 1, dtype: torch.dtype = torch.bfloat16, seed: Optional[int] = None):
    """(x ``[B, N, 1024]`` ~ N(0, 1) in ``dtype``, positions) for a full layer forward."""
    g = _gen(BASE_SEED + views if seed is None else seed)
    x = torch.randn(batch, views * TOKENS_PER_VIEW, DIM, generator=g).to(dtype)
    return x, patch_positions(views, batch)


def init_layer_(layer: torch.nn.Module, seed: int = BASE_SEED) -> torch.nn.Module:
    """Random-init a SparseGlobalAttention in place (no checkpoint exists offline): linear
    weights ~ N(0, 1/dim) (unit-variance projections), biases ~ N(0, 0.02), LayerNorm
    gains 1 + N(0, 0.1), the indexer gate bias 1 (its reference init, ``indexer.py:63-68``)
    with weights ~ N(0, 0.25/dim)."""
    g = _gen(seed)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if p.dim() == 2:
                scale = (0.25 if "w_proj" in name else 1.0) / p.shape[1] ** 0.5
                p.copy_(torch.randn(p.shape, generator=g) * scale)
            elif "norm" in name and name.endswith("weight"):
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g))
            elif "w_proj" in name:
                p.fill_(1.0)
            else:
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
    return layer
