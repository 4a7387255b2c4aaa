"""Lightning-indexer score + exact top-k on gfx950: the drop-in for the reference module
``easyvolcap/utils/custom_indexer/sparse_topk_indexer.py``.

``sparse_topk_indexer_func(q, k, w, mask, topk, softmax_scale, block_k, merge_blocks=0,
view_bias_data=None) -> (topk_indices int32 [B,T,K], topk_scores q.dtype [B,T,K])`` with
``K = min(topk, S)``, differentiable w.r.t. q, k, w through ``topk_scores`` (reference
``:2047-2106,2188-2253``). The index order inside a row is unspecified (the reference uses
``sorted=False``). ``block_k`` and ``merge_blocks`` are the reference's tuning hints for its
blockwise host loop; this implementation has no such loop and ignores them.

``sparse_topk_indexer_inference_func`` is the no-autograd entry with the call signature
used by the reference caller (``easyvolcap/official_vggt/layers/indexer.py:570-581``);
the reference package leaves it ``None`` (``custom_indexer/__init__.py:7``).

Inputs: q ``[B,T,Hi,Di]``, k ``[B,S,Hi,Di]``, w ``[B,S,Hi]`` in one 16-bit float dtype on
the GPU; mask: ``None``, an empty tensor, or an additive ``[B,T,S]`` (broadcast from
``[T,S]``/``[1,T,S]``). Supported: ``Di = 64``, ``Hi in {1,2,4,8}``, ``K <= 2048``.
``view_bias_data`` (the soft view-bias training kernel) is not implemented.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from .. import _lib

__all__ = ["sparse_topk_indexer_func", "sparse_topk_indexer_inference_func", "SparseTopkIndexerFunc"]

FLAG_TAU_PLUS_INF = 1
FLAG_TAU_MINUS_INF = 2
FLAG_FORCE_WIDE = 4


def _normalize_mask(mask: Optional[torch.Tensor], bsz: int, tgt_len: int, src_len: int, dtype):
    # reference: sparse_topk_indexer.py:2201-2202 (empty -> None), :1299-1300 (cast to q dtype)
    if mask is None or mask.numel() == 0:
        return None
    if mask.dim() == 2:
        mask = mask.unsqueeze(0)
    if mask.dim() != 3 or mask.shape[-2:] != (tgt_len, src_len) or mask.shape[0] not in (1, bsz):
        raise ValueError(f"mask shape {tuple(mask.shape)} does not match ({bsz}, {tgt_len}, {src_len})")
    return mask.to(dtype).expand(bsz, tgt_len, src_len).contiguous()


def _check(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor):
    if q.dim() != 4 or k.dim() != 4 or w.dim() != 3:
        raise ValueError("q/k/w must be [B,T,H,D], [B,S,H,D], [B,S,H]")
    bsz, tgt_len, n_heads, head_dim = q.shape
    if k.shape[0] != bsz or k.shape[2] != n_heads or k.shape[3] != head_dim:
        raise ValueError(f"k shape {tuple(k.shape)} mismatches q {tuple(q.shape)}")
    if tuple(w.shape) != (bsz, k.shape[1], n_heads):
        raise ValueError(f"w shape {tuple(w.shape)} mismatches q {tuple(q.shape)} and k {tuple(k.shape)}")
    if not (q.dtype == k.dtype == w.dtype):
        raise TypeError("q, k and w must have the same dtype")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"the HIP indexer takes bfloat16 or float16 inputs, got {q.dtype}")
    if not (q.is_cuda and k.is_cuda and w.is_cuda):
        raise ValueError("q, k and w must be GPU tensors")
    if head_dim != 64 or n_heads not in (1, 2, 4, 8):
        raise NotImplementedError(f"indexer heads x dim {n_heads} x {head_dim} not built (1/2/4/8 x 64)")


def indexer_topk_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    mask: Optional[torch.Tensor],
    topk: int,
    softmax_scale: Optional[float],
    flags: int = 0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Launches gw_indexer_topk_fwd on the current stream; returns (indices, scores)."""
    _check(q, k, w)
    q = q.contiguous()
    k = k.contiguous()
    w = w.contiguous()
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(head_dim)
    if not softmax_scale > 0:
        raise ValueError(f"softmax_scale must be positive, got {softmax_scale}")
    mask = _normalize_mask(mask, bsz, tgt_len, src_len, q.dtype)
    kk = min(int(topk), int(src_len))
    if kk <= 0:
        raise ValueError(f"topk must be positive (got topk={topk}, S={src_len})")
    idx = torch.empty((bsz, tgt_len, kk), device=q.device, dtype=torch.int32)
    scores = torch.empty((bsz, tgt_len, kk), device=q.device, dtype=q.dtype)
    if bsz == 0 or tgt_len == 0:
        return idx, scores
    lib = _lib.load()
    ws_bytes = int(lib.gw_indexer_topk_workspace_size(bsz, tgt_len, src_len, kk))
    ws = torch.empty(max(ws_bytes, 16), device=q.device, dtype=torch.uint8)
    rc = lib.gw_indexer_topk_fwd(
        _lib.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), w.data_ptr(), _lib.ptr(mask),
        bsz, tgt_len, src_len, n_heads, head_dim, kk, float(softmax_scale), int(flags),
        idx.data_ptr(), scores.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
    )
    _lib.check(rc, "gw_indexer_topk_fwd")
    return idx, scores


def indexer_topk_backward(q, k, w, topk_indices, grad_scores, softmax_scale):
    from . import _backward

    return _backward.indexer_topk_backward(q, k, w, topk_indices, grad_scores, softmax_scale)


class SparseTopkIndexerFunc(torch.autograd.Function):
    """Autograd wrapper (reference ``sparse_topk_indexer.py:2047-2106``)."""

    @staticmethod
    def forward(ctx, q, k, w, mask, topk, softmax_scale, block_k, merge_blocks):
        q = q.contiguous()
        k = k.contiguous()
        w = w.contiguous()
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])
        with torch.no_grad():
            topk_indices, topk_scores = indexer_topk_forward(q, k, w, mask, topk, softmax_scale)
        ctx.save_for_backward(q, k, w, topk_indices)
        ctx.softmax_scale = float(softmax_scale)
        ctx.mark_non_differentiable(topk_indices)
        return topk_indices, topk_scores

    @staticmethod
    def backward(ctx, grad_indices, grad_scores):
        q, k, w, topk_indices = ctx.saved_tensors
        if grad_scores is None:
            return None, None, None, None, None, None, None, None
        if grad_scores.stride(-1) != 1:
            grad_scores = grad_scores.contiguous()
        dq, dk, dw = indexer_topk_backward(q, k, w, topk_indices, grad_scores, ctx.softmax_scale)
        return dq, dk, dw, None, None, None, None, None


def sparse_topk_indexer_func(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    mask: Optional[torch.Tensor],
    topk: int,
    softmax_scale: Optional[float],
    block_k: int,
    merge_blocks: int = 0,
    view_bias_data: Optional[dict] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Drop-in for the reference ``sparse_topk_indexer_func`` (``:2188-2253``)."""
    if view_bias_data is not None:
        raise NotImplementedError("view_bias_data (soft view-bias kernel) is not supported by the HIP indexer")
    if mask is not None and mask.numel() == 0:
        mask = None
    return SparseTopkIndexerFunc.apply(q, k, w, mask, topk, softmax_scale, block_k, merge_blocks)


@torch.no_grad()
def sparse_topk_indexer_inference_func(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    mask: Optional[torch.Tensor],
    topk: int,
    softmax_scale: Optional[float],
    block_k: int = 256,
    merge_blocks: int = 0,
    outer_query_chunk: int = 0,
    return_scores: bool = True,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Inference-only entry with the caller's signature (reference ``indexer.py:570-581``).
    ``outer_query_chunk`` is a memory hint of the reference; the HIP path never holds
    more than the per-query candidate lists, so it is ignored."""
    idx, scores = indexer_topk_forward(q, k, w, mask, topk, softmax_scale)
    return idx, (scores if return_scores else None)
