"""VGGT-style alternating-attention aggregator around the sparse global-attention layer.

The host path of the reference ``Aggregator`` (``easyvolcap/official_vggt/models/
aggregator.py:54-722``) with the pieces its sparse global blocks need:

* frame blocks (dense attention within each view) and global blocks (attention over all
  views' tokens) alternate, 24 of each (``aa_order = [frame, global]``, ``:552-566``);
* global blocks listed in ``indexer_layers`` (VGGT: 9-19) are sparse: their attention is
  ``dsa_layer.SparseGlobalAttention`` (fused projection, layer glue, indexer top-k, sparse
  attention), the others dense;
* ``reuse_topk_groups`` (``:158-164,327-362,401-423``): a layer mapped to a source layer
  reuses the source's top-k indices of the same forward and skips its own indexer;
* a VGGT patch embedding: the DINOv2-style ViT-L/14 with 4 register tokens (conv patchify,
  class + register tokens, learned position embedding, 24 dense blocks, final norm), then
  the aggregator's camera and register tokens (``:504-526``, ``:723-746``) and 2D rotary
  positions (patches at (row + 1, col + 1), special tokens at (0, 0));
* optional HIP-graph capture of the whole forward (the reference captures its DSA
  attention "fullchain", ``dsa_attention.py:1600-1675``): ``AggregatorGraph`` records
  one replayable graph per input shape on static buffers.

Weights are random (no checkpoint is available offline); parameter names follow the
reference (``frame_blocks.{i}``, ``global_blocks.{i}`` with ``norm1``, ``attn``, ``ls1``,
``norm2``, ``mlp.fc1/fc2``, ``ls2``). Everything runs in bf16 (or fp16) on the GPU; dense
attention uses torch's fused scaled-dot-product kernels (flash / memory-efficient only:
the unfused path is disabled). The dense layers' q/k LayerNorm + RoPE use the same HIP
glue kernel as the sparse layers.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Set, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import dsa_layer, source_downsample

__all__ = ["parse_indexer_layers", "parse_reuse_topk_groups", "slice_expand_and_flatten", "Aggregator",
           "AggregatorGraph"]

_RESNET_MEAN = (0.485, 0.456, 0.406)
_RESNET_STD = (0.229, 0.224, 0.225)


def parse_indexer_layers(spec) -> Optional[Set[int]]:
    """Layer set from ``"9-19"``, ``"1,3,5-7"``, a list, ``"all"``/``"*"`` (None = every
    layer) or None; reference ``Aggregator._parse_indexer_layers`` (``aggregator.py:267-292``)."""
    if spec is None:
        return None
    if isinstance(spec, str):
        text = spec.strip()
        if not text:
            return set()
        if text.lower() in ("all", "*"):
            return None
        out: Set[int] = set()
        for item in (t.strip() for t in text.split(",") if t.strip()):
            if "-" in item:
                left, right = (t.strip() for t in item.split("-", 1))
                if left and right:
                    out.update(range(int(left), int(right) + 1))
                    continue
            out.add(int(item))
        return out
    if isinstance(spec, (list, tuple, set)):
        return {int(v) for v in spec}
    return None


def parse_reuse_topk_groups(groups) -> Optional[Dict[int, int]]:
    """``{layer: source}`` from items ``"src:layers"`` (layers as in
    :func:`parse_indexer_layers`) and ``"a-b"`` (source min(a, b) for the layers above it up
    to max(a, b)); bare integers are ignored. Reference ``_parse_reuse_topk_groups``
    (``aggregator.py:327-362``)."""
    if groups is None:
        return None
    if isinstance(groups, str):
        text = groups.strip()
        if not text:
            return {}
        items = [t.strip() for t in text.split(",") if t.strip()]
    elif isinstance(groups, (list, tuple, set)):
        items = [str(t).strip() for t in groups if str(t).strip()]
    else:
        return None
    out: Dict[int, int] = {}
    for item in items:
        if ":" in item:
            src_text, layers_text = item.split(":", 1)
            src = int(src_text.strip())
            layers = parse_indexer_layers(layers_text.strip())
            if layers is None:
                continue
            for layer in layers:
                if int(layer) != src:
                    out[int(layer)] = src
            continue
        if "-" in item:
            left, right = item.split("-", 1)
            src, hi = int(left.strip()), int(right.strip())
            if hi < src:
                src, hi = hi, src
            for layer in range(src + 1, hi + 1):
                out[layer] = src
            continue
        int(item)  # a bare layer id is valid syntax and names no reuse
    return out


def slice_expand_and_flatten(token: torch.Tensor, B: int, S: int) -> torch.Tensor:
    """``[1, 2, X, C]`` -> ``[B*S, X, C]``: slot 0 for the first view, slot 1 for the others
    (reference ``aggregator.py:723-746``)."""
    first = token[:, 0:1].expand(B, 1, *token.shape[2:])
    others = token[:, 1:].expand(B, S - 1, *token.shape[2:])
    return torch.cat([first, others], dim=1).reshape(B * S, *token.shape[2:])


def _sdpa(q, k, v):
    from torch.nn.attention import SDPBackend, sdpa_kernel

    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v)


class LayerScale(nn.Module):
    def __init__(self, dim: int, init_values: float = 0.01):
        super().__init__()
        self.gamma = nn.Parameter(init_values * torch.ones(dim))

    def forward(self, x):
        return x * self.gamma


class Mlp(nn.Module):
    def __init__(self, dim: int, hidden: int):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden)
        self.act = nn.GELU()
        self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x):
        return self.fc2(self.act(self.fc1(x)))


class DenseAttention(nn.Module):
    """Reference ``layers/attention.py:38-98`` (fused path): qkv, q/k LayerNorm, 2D RoPE,
    scaled-dot-product attention, proj. q/k LayerNorm + RoPE run in the HIP glue kernel."""

    def __init__(self, dim: int, num_heads: int, qk_norm: bool, rope_base: Optional[float]):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.qkv = nn.Linear(dim, 3 * dim)
        self.q_norm = nn.LayerNorm(self.head_dim) if qk_norm else nn.Identity()
        self.k_norm = nn.LayerNorm(self.head_dim) if qk_norm else nn.Identity()
        self.proj = nn.Linear(dim, dim)
        self.rope_base = rope_base
        self.layout = dsa_layer.GlueLayout(num_heads, self.head_dim, 0, 64)

    def forward(self, x, pos=None, rope_len=None):
        B, N, C = x.shape
        y = self.qkv(x)
        use_glue = not (isinstance(self.q_norm, nn.Identity) and (self.rope_base is None or pos is None))
        if use_glue:
            q, k, v, _, _, _ = dsa_layer.dsa_glue_forward(
                y, self.layout, dsa_layer._ln_params(self.q_norm), dsa_layer._ln_params(self.k_norm),
                (None, None), 1e-5, pos if self.rope_base else None, self.rope_base or 100.0, rope_len)
        else:
            q, k, v = y.view(B, N, 3, self.num_heads, self.head_dim).unbind(2)
        o = _sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
        return self.proj(o.transpose(1, 2).reshape(B, N, C))


class Block(nn.Module):
    """``x + ls1(attn(norm1(x))) -> + ls2(mlp(norm2(x)))`` (reference ``layers/block.py:28-99``);
    ``attn`` is dense or sparse."""

    def __init__(self, dim: int, num_heads: int, mlp_ratio: float, qk_norm: bool, rope_base: Optional[float],
                 sparse: bool = False, topk: int = 1024, init_values: float = 0.01, score_dtype=None):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim)
        self.sparse = sparse
        if sparse:
            self.attn = dsa_layer.SparseGlobalAttention(dim, num_heads, qk_norm=qk_norm, rope_base=rope_base,
                                                        topk=topk, score_dtype=score_dtype)
        else:
            self.attn = DenseAttention(dim, num_heads, qk_norm, rope_base)
        self.ls1 = LayerScale(dim, init_values)
        self.norm2 = nn.LayerNorm(dim)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        self.ls2 = LayerScale(dim, init_values)

    timing = None  # a list to collect (start, end) HIP events around the attention call

    def forward(self, x, pos=None, rope_len=None, topk_indices=None, source_downsample=None):
        idx = None
        h = self.norm1(x)
        ev = None
        if self.timing is not None:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        if self.sparse:
            a, idx = self.attn(h, pos, return_topk=True, topk_indices=topk_indices, rope_len=rope_len,
                               source_downsample=source_downsample)
        else:
            a = self.attn(h, pos, rope_len)
        if ev is not None:
            ev[1].record()
            self.timing.append(ev)
        x = x + self.ls1(a)
        x = x + self.ls2(self.mlp(self.norm2(x)))
        return x, idx


class PatchEmbedViT(nn.Module):
    """DINOv2-style ViT-L/14 with registers as the patch embedding (``patch_embed =
    dinov2_vitl14_reg``, ``aggregator.py:399-470``): conv patchify, class + register tokens,
    learned position embedding for a 37 x 37 grid, ``depth`` dense blocks without RoPE,
    final LayerNorm; returns the normed patch tokens ``[B*S, 1369, dim]``."""

    def __init__(self, dim: int = 1024, depth: int = 24, num_heads: int = 16, patch: int = 14, grid: int = 37,
                 num_register_tokens: int = 4):
        super().__init__()
        self.patch = patch
        self.grid = grid
        self.num_register_tokens = num_register_tokens
        self.proj = nn.Conv2d(3, dim, patch, patch)
        self.cls_token = nn.Parameter(torch.zeros(1, 1, dim))
        self.register_tokens = nn.Parameter(torch.zeros(1, num_register_tokens, dim))
        self.pos_embed = nn.Parameter(torch.zeros(1, grid * grid + 1, dim))
        self.blocks = nn.ModuleList(Block(dim, num_heads, 4.0, False, None, init_values=1e-5) for _ in range(depth))
        self.norm = nn.LayerNorm(dim)

    def forward(self, images):
        # The stride-14 14 x 14 convolution as one GEMM over (channel, row, column)-ordered
        # patches, the order of the conv weight [dim, 3, 14, 14].
        n, c, h, w = images.shape
        g, ps = self.grid, self.patch
        if h != g * ps or w != g * ps:
            raise ValueError(f"images must be {g * ps} x {g * ps} (a {g} x {g} patch grid)")
        patches = images.reshape(n, c, g, ps, g, ps).permute(0, 2, 4, 1, 3, 5).reshape(n, g * g, c * ps * ps)
        x = F.linear(patches, self.proj.weight.reshape(self.proj.out_channels, -1), self.proj.bias)
        x = torch.cat([self.cls_token.expand(x.shape[0], -1, -1), x], 1) + self.pos_embed
        x = torch.cat([x[:, :1], self.register_tokens.expand(x.shape[0], -1, -1), x[:, 1:]], 1)
        for blk in self.blocks:
            x, _ = blk(x)
        return self.norm(x)[:, 1 + self.num_register_tokens:]


class SpecialTokens(nn.Module):
    def __init__(self, dim: int, num_register_tokens: int):
        super().__init__()
        self.camera_token = nn.Parameter(torch.randn(1, 2, 1, dim))
        self.register_token = nn.Parameter(torch.randn(1, 2, num_register_tokens, dim))


class Aggregator(nn.Module):
    """``forward(images [B, S, 3, 518, 518] in [0, 1]) -> (list of depth tensors [B, S, P,
    2*dim], patch_start_idx)`` (reference ``Aggregator.forward``, ``aggregator.py:472-597``)."""

    def __init__(self, dim: int = 1024, depth: int = 24, num_heads: int = 16, mlp_ratio: float = 4.0,
                 num_register_tokens: int = 4, qk_norm: bool = True, rope_freq: float = 100.0,
                 indexer_layers="9-19", reuse_topk_groups=None, topk: int = 1024, patch_depth: int = 24,
                 img_size: int = 518, patch_size: int = 14, source_downsample_factor: int = 1,
                 source_downsample_options: Optional[Dict] = None, score_dtype=None):
        super().__init__()
        # score_dtype: the sparse layers' indexer and attention dtype (the reference preset's
        # indexer_cfg "score_dtype", geoweave/configs/vggt.json:35); None = the activations'.
        # Approximate coarse selection in the sparse layers (off at factor 1, the reference
        # default; dsa_attention.py:122-132): the per-forward layout is filled in below.
        self.source_downsample_factor = int(source_downsample_factor)
        self.source_downsample_options = dict(source_downsample_options or {})
        self.depth = depth
        self.patch_size = patch_size
        grid = img_size // patch_size
        self.patch_embed = PatchEmbedViT(dim, patch_depth, num_heads, patch_size, grid, num_register_tokens)
        self.special_tokens = SpecialTokens(dim, num_register_tokens)
        self.patch_start_idx = 1 + num_register_tokens
        rope = rope_freq if rope_freq and rope_freq > 0 else None
        sparse = parse_indexer_layers(indexer_layers)
        self.sparse_layers = set(range(depth)) if sparse is None else {i for i in sparse if 0 <= i < depth}
        reuse = parse_reuse_topk_groups(reuse_topk_groups) or {}
        self.reuse_topk_source_by_layer = {l: s for l, s in reuse.items()
                                           if 0 <= l < depth and 0 <= s < depth and l != s
                                           and l in self.sparse_layers and s in self.sparse_layers}
        self.frame_blocks = nn.ModuleList(Block(dim, num_heads, mlp_ratio, qk_norm, rope) for _ in range(depth))
        self.global_blocks = nn.ModuleList(
            Block(dim, num_heads, mlp_ratio, qk_norm, rope, sparse=i in self.sparse_layers, topk=topk,
                  score_dtype=score_dtype)
            for i in range(depth))
        self.register_buffer("_resnet_mean", torch.tensor(_RESNET_MEAN).view(1, 1, 3, 1, 1), persistent=False)
        self.register_buffer("_resnet_std", torch.tensor(_RESNET_STD).view(1, 1, 3, 1, 1), persistent=False)

    def positions(self, B: int, S: int, grid: int, device) -> torch.Tensor:
        ys, xs = torch.meshgrid(torch.arange(grid, device=device), torch.arange(grid, device=device), indexing="ij")
        patch = torch.stack([ys.reshape(-1), xs.reshape(-1)], -1) + 1
        special = torch.zeros(self.patch_start_idx, 2, dtype=patch.dtype, device=device)
        return torch.cat([special, patch], 0).to(torch.int32).expand(B * S, -1, -1)

    @torch.no_grad()
    def forward(self, images: torch.Tensor) -> Tuple[List[torch.Tensor], int]:
        B, S, C_in, H, W = images.shape
        if C_in != 3:
            raise ValueError(f"expected 3 input channels, got {C_in}")
        dtype = self.frame_blocks[0].norm1.weight.dtype
        x = ((images - self._resnet_mean) / self._resnet_std).to(dtype).reshape(B * S, C_in, H, W)
        patch_tokens = self.patch_embed(x)
        tokens = torch.cat([slice_expand_and_flatten(self.special_tokens.camera_token, B, S),
                            slice_expand_and_flatten(self.special_tokens.register_token, B, S),
                            patch_tokens], dim=1)
        P, C = tokens.shape[1], tokens.shape[2]
        grid = H // self.patch_size
        pos = self.positions(B, S, grid, images.device)
        rope_len = grid + 1  # positions run over [0, grid]: no host read of max(pos)
        pos_global = pos.reshape(B, S * P, 2)
        cached: Dict[int, torch.Tensor] = {}
        sources = set(self.reuse_topk_source_by_layer.values())
        sd = None
        if self.source_downsample_factor > 1:
            sd = source_downsample.SourceDownsample(tokens_per_view=P, num_views=S,
                                                    patch_start_idx=self.patch_start_idx,
                                                    factor=self.source_downsample_factor, grid_h=grid, grid_w=grid,
                                                    **self.source_downsample_options)
        outputs = []
        for i in range(self.depth):
            tokens, _ = self.frame_blocks[i](tokens.reshape(B * S, P, C), pos, rope_len)
            frame_out = tokens.reshape(B, S, P, C)
            blk = self.global_blocks[i]
            reuse = cached.get(self.reuse_topk_source_by_layer.get(i, -1)) if blk.sparse else None
            tokens, idx = blk(tokens.reshape(B, S * P, C), pos_global, rope_len, topk_indices=reuse,
                              source_downsample=sd)
            if blk.sparse and i in sources:
                cached[i] = idx
            outputs.append(torch.cat([frame_out, tokens.reshape(B, S, P, C)], dim=-1))
        return outputs, self.patch_start_idx


def random_init_(model: Aggregator, seed: int = 20261201) -> Aggregator:
    """Random-init the aggregator in place (no checkpoint exists offline): matrices and
    convolution kernels ~ N(0, 1/fan_in), LayerScale gammas 0.1, LayerNorm gains
    1 + N(0, 0.1), the indexer gate bias 1 (its reference init, ``indexer.py:63-68``), other
    vectors ~ N(0, 0.02). Draws on the parameters' device."""
    torch.manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() >= 2:
                p.normal_(0.0, p[0].numel() ** -0.5)
            elif name.endswith("gamma"):
                p.fill_(0.1)
            elif "norm" in name and name.endswith("weight"):
                p.normal_(1.0, 0.1)
            elif "w_proj" in name:
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02)
    return model


class AggregatorGraph:
    """One HIP graph per input shape replaying the whole aggregator forward on static
    buffers (the reference's CUDA-graph "fullchain" path, ``dsa_attention.py:1600-1675``,
    applied to the whole stack). ``__call__(images)`` copies into the static input,
    replays, and returns the static outputs (valid until the next call)."""

    def __init__(self, model: Aggregator, warmup: int = 1):
        self.model = model
        self.warmup = warmup
        self.entries = {}

    def __call__(self, images: torch.Tensor):
        key = (tuple(images.shape), images.dtype, images.device)
        entry = self.entries.get(key)
        if entry is None:
            static_in = images.clone()
            side = torch.cuda.Stream(device=images.device)
            side.wait_stream(torch.cuda.current_stream(images.device))
            with torch.cuda.stream(side):
                for _ in range(self.warmup):
                    self.model(static_in)
            torch.cuda.current_stream(images.device).wait_stream(side)
            torch.cuda.synchronize(images.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                static_out = self.model(static_in)
            entry = (graph, static_in, static_out)
            self.entries[key] = entry
        graph, static_in, static_out = entry
        static_in.copy_(images)
        graph.replay()
        return static_out
