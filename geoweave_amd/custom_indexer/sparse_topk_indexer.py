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

Inputs: q ``[B,T,Hi,Di]``, k ``[B,S,Hi,Di]``, w ``[B,S,Hi]`` in one float dtype on the GPU:
bfloat16 or float16 (bf16/fp16 matrix-core products, fp32 accumulation) or float32 (fp32
matrix-core products; the reference computes in ``q.dtype`` too, ``:1293``, and its caller
may cast to ``score_dtype="float32"``, ``indexer.py:321-326``); scores come back in
``q.dtype``. mask: ``None``, an empty tensor, or an additive ``[B,T,S]`` (broadcast from
``[T,S]``/``[1,T,S]``), cast to ``q.dtype`` as the reference does (``:1299-1300``).
Supported: ``Di <= 64`` (the kernels take 64; smaller head dims run zero-padded to it),
``Hi <= 8`` (``<= 4`` in float32; the kernels take 1, 2, 4 or 8 heads, other counts run
with zero heads appended), any ``K`` (one whose expected candidates would overflow the
8,192 candidate slots scores every row over every key and selects it exactly).

``view_bias_data`` (the soft view-bias training kernel, reference ``:2108-2186``): a dict
with ``q_view_ids`` ``[B,T]``/``[T]``, ``s_view_ids`` ``[B,S]``/``[S]`` and ``view_bias``
``[B,Vq,Vs]``/``[Vq,Vs]``; every score gets ``view_bias[b, q_view_ids[b,t],
s_view_ids[b,s]]`` added after the mask, inside the HIP top-k (``gw_indexer_topk_fwd_view_bias``),
and ``view_bias`` receives the gradient of the selected scores (``gw_indexer_view_bias_bwd_rows``
and a one-hot product over query views). A dict missing any of the three keys counts as
no view bias, as in the reference (``:635-636``).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from .. import _lib

__all__ = ["sparse_topk_indexer_func", "sparse_topk_indexer_inference_func", "SparseTopkIndexerFunc",
           "SparseTopkIndexerViewBiasFunc"]

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


# The kernels' head dim. Smaller ones (the reference takes any, sparse_topk_indexer.py:777,
# 1143) run on q and k zero-padded to it: padded dims add nothing to q.k, and the backward's
# dq, dk are cut back to the input's head dim.
KERNEL_HEAD_DIM = 64


def pad_head_dim(x: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.pad(x, (0, KERNEL_HEAD_DIM - x.shape[-1]))


# The kernels' head counts. Other counts up to the largest (the reference's block kernel takes
# any, masking heads past n_heads, sparse_topk_indexer.py:1009,1029,1142) run with zero heads
# appended: a zero head (q = k = 0, w = 0) adds w relu(q.k) = 0 to every score, and the
# backward's gradients of the real heads do not depend on it (they are cut back).
KERNEL_HEADS = (1, 2, 4, 8)
KERNEL_HEADS_FP32 = (1, 2, 4)


def kernel_heads(n_heads: int, dtype: torch.dtype) -> Optional[int]:
    """The built head count that ``n_heads`` runs as (None: above every built count)."""
    built = KERNEL_HEADS_FP32 if dtype == torch.float32 else KERNEL_HEADS
    return next((h for h in built if h >= n_heads), None)


def pad_heads(x: torch.Tensor, n_heads: int) -> torch.Tensor:
    """q, k ``[B, T, H, D]`` or w ``[B, S, H]`` with zero heads appended up to ``n_heads``."""
    extra = n_heads - x.shape[2]
    return torch.nn.functional.pad(x, (0, 0, 0, extra) if x.dim() == 4 else (0, extra))


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
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"the HIP indexer takes bfloat16, float16 or float32 inputs, got {q.dtype}")
    if not (q.is_cuda and k.is_cuda and w.is_cuda):
        raise ValueError("q, k and w must be GPU tensors")
    if not 1 <= head_dim <= 64 or n_heads < 1 or kernel_heads(n_heads, q.dtype) is None:
        raise NotImplementedError(f"indexer heads x dim {n_heads} x {head_dim} not built (up to 8 heads, "
                                  f"4 in float32, x up to 64 dims)")


def _normalize_view_bias_data(view_bias_data: Optional[dict], bsz: int, tgt_len: int, src_len: int,
                              device, dtype) -> Optional[dict]:
    """The reference's shape rules (``sparse_topk_indexer.py:621-659``): 1-D id vectors and a
    2-D table gain a batch dimension, a batch of one is broadcast to ``bsz``; ids become
    int64 and the table takes q's dtype. Missing keys: None (no view bias)."""
    if view_bias_data is None:
        return None
    q_ids = view_bias_data.get("q_view_ids", None)
    s_ids = view_bias_data.get("s_view_ids", None)
    table = view_bias_data.get("view_bias", None)
    if q_ids is None or s_ids is None or table is None:
        return None
    q_ids = q_ids.unsqueeze(0) if q_ids.dim() == 1 else q_ids
    s_ids = s_ids.unsqueeze(0) if s_ids.dim() == 1 else s_ids
    table = table.unsqueeze(0) if table.dim() == 2 else table
    if q_ids.size(0) == 1 and bsz > 1:
        q_ids = q_ids.expand(bsz, -1)
    if s_ids.size(0) == 1 and bsz > 1:
        s_ids = s_ids.expand(bsz, -1)
    if table.size(0) == 1 and bsz > 1:
        table = table.expand(bsz, -1, -1)
    if tuple(q_ids.shape) != (bsz, tgt_len):
        raise ValueError(f"q_view_ids shape {tuple(q_ids.shape)} mismatches ({bsz}, {tgt_len})")
    if tuple(s_ids.shape) != (bsz, src_len):
        raise ValueError(f"s_view_ids shape {tuple(s_ids.shape)} mismatches ({bsz}, {src_len})")
    if table.dim() != 3 or int(table.shape[0]) != int(bsz):
        raise ValueError(f"view_bias shape {tuple(table.shape)} mismatches batch {bsz}")
    return dict(q_view_ids=q_ids.to(device=device, dtype=torch.long),
                s_view_ids=s_ids.to(device=device, dtype=torch.long),
                view_bias=table.to(device=device, dtype=dtype))


def _view_ids_int32(q_view_ids: torch.Tensor, s_view_ids: torch.Tensor, n_q_views: int, n_s_views: int):
    """int32 contiguous ids, checked against the table (an out-of-range id is an indexing
    error in the reference's gather, ``indexer.py:519``; the kernels clamp, this raises)."""
    qv = q_view_ids.to(torch.int32).contiguous()
    sv = s_view_ids.to(torch.int32).contiguous()
    lo_q, hi_q, lo_s, hi_s = torch.stack([qv.min(), qv.max(), sv.min(), sv.max()]).tolist()
    if lo_q < 0 or hi_q >= n_q_views or lo_s < 0 or hi_s >= n_s_views:
        raise IndexError(f"view ids out of range: q in [{lo_q}, {hi_q}] for {n_q_views} query views, "
                         f"s in [{lo_s}, {hi_s}] for {n_s_views} key views")
    return qv, sv


def indexer_topk_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    mask: Optional[torch.Tensor],
    topk: int,
    softmax_scale: Optional[float],
    flags: int = 0,
    view_bias: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Launches gw_indexer_topk_fwd (gw_indexer_topk_fwd_view_bias when ``view_bias`` =
    (q_view_ids int32 [B,T], s_view_ids int32 [B,S], table [B,Vq,Vs] in q's dtype), all
    contiguous) on the current stream; returns (indices, scores)."""
    _check(q, k, w)
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(head_dim)
    if head_dim != KERNEL_HEAD_DIM:
        q, k, head_dim = pad_head_dim(q), pad_head_dim(k), KERNEL_HEAD_DIM
    built_heads = kernel_heads(n_heads, q.dtype)
    if built_heads != n_heads:
        q, k, w, n_heads = pad_heads(q, built_heads), pad_heads(k, built_heads), pad_heads(w, built_heads), built_heads
    q = q.contiguous()
    k = k.contiguous()
    w = w.contiguous()
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
    if view_bias is not None:
        qv, sv, table = view_bias
        rc = lib.gw_indexer_topk_fwd_view_bias(
            _lib.dtype_code(q.dtype, allow_fp32=True), q.data_ptr(), k.data_ptr(), w.data_ptr(), _lib.ptr(mask),
            table.data_ptr(), qv.data_ptr(), sv.data_ptr(), int(table.shape[1]), int(table.shape[2]),
            bsz, tgt_len, src_len, n_heads, head_dim, kk, float(softmax_scale), int(flags),
            idx.data_ptr(), scores.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
        )
        _lib.check(rc, "gw_indexer_topk_fwd_view_bias")
        return idx, scores
    rc = lib.gw_indexer_topk_fwd(
        _lib.dtype_code(q.dtype, allow_fp32=True), q.data_ptr(), k.data_ptr(), w.data_ptr(), _lib.ptr(mask),
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


def view_bias_backward(topk_indices: torch.Tensor, grad_scores: torch.Tensor, q_view_ids: torch.Tensor,
                       s_view_ids: torch.Tensor, shape, dtype) -> torch.Tensor:
    """grad of view_bias ``[B, Vq, Vs]`` from the selected scores' gradient (reference
    ``_scatter_view_bias_grad``, ``sparse_topk_indexer.py:898-932``): fp32 sums, cast to the
    table's dtype. Row sums over key views on the GPU (``gw_indexer_view_bias_bwd_rows``,
    fixed order), then per batch the one-hot matrix of query views times the row sums."""
    bsz, tgt_len, kk = topk_indices.shape
    _, n_q, n_s = shape
    src_len = int(s_view_ids.shape[1])
    rows = torch.empty((bsz, tgt_len, n_s), device=grad_scores.device, dtype=torch.float32)
    if bsz * tgt_len > 0:
        g = grad_scores.to(topk_indices.device).contiguous()
        if g.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise TypeError(f"grad_scores must be bfloat16, float16 or float32, got {g.dtype}")
        rc = _lib.load().gw_indexer_view_bias_bwd_rows(
            _lib.dtype_code(g.dtype, allow_fp32=True), topk_indices.contiguous().data_ptr(), g.data_ptr(), s_view_ids.data_ptr(),
            bsz, tgt_len, src_len, kk, n_s, rows.data_ptr(), _lib.stream_handle(g.device))
        _lib.check(rc, "gw_indexer_view_bias_bwd_rows")
    onehot = torch.nn.functional.one_hot(q_view_ids.long(), n_q).to(torch.float32)  # [B, T, Vq]
    grad = torch.bmm(onehot.transpose(1, 2).contiguous(), rows)  # [B, Vq, Vs]
    return grad.to(dtype)


class SparseTopkIndexerViewBiasFunc(torch.autograd.Function):
    """Autograd wrapper with the soft view bias (reference ``sparse_topk_indexer.py:
    2108-2186``): gradients for q, k, w (as ``SparseTopkIndexerFunc``) and for the table."""

    @staticmethod
    def forward(ctx, q, k, w, mask, q_view_ids, s_view_ids, view_bias, topk, softmax_scale, block_k, merge_blocks):
        q = q.contiguous()
        k = k.contiguous()
        w = w.contiguous()
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])
        table = view_bias.contiguous()
        qv, sv = _view_ids_int32(q_view_ids, s_view_ids, int(table.shape[1]), int(table.shape[2]))
        with torch.no_grad():
            topk_indices, topk_scores = indexer_topk_forward(q, k, w, mask, topk, softmax_scale,
                                                             view_bias=(qv, sv, table))
        ctx.save_for_backward(q, k, w, topk_indices, qv, sv)
        ctx.softmax_scale = float(softmax_scale)
        ctx.view_bias_shape = tuple(int(x) for x in view_bias.shape)
        ctx.view_bias_dtype = view_bias.dtype
        ctx.mark_non_differentiable(topk_indices)
        return topk_indices, topk_scores

    @staticmethod
    def backward(ctx, grad_indices, grad_scores):
        q, k, w, topk_indices, qv, sv = ctx.saved_tensors
        if grad_scores is None:
            return (None,) * 11
        if grad_scores.stride(-1) != 1:
            grad_scores = grad_scores.contiguous()
        dq, dk, dw = indexer_topk_backward(q, k, w, topk_indices, grad_scores, ctx.softmax_scale)
        grad_view_bias = None
        if ctx.needs_input_grad[6]:
            grad_view_bias = view_bias_backward(topk_indices, grad_scores, qv, sv, ctx.view_bias_shape,
                                                ctx.view_bias_dtype)
        return dq, dk, dw, None, None, None, grad_view_bias, None, None, None, None


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
    if mask is not None and mask.numel() == 0:
        mask = None
    if view_bias_data is not None:
        _check(q, k, w)
        norm = _normalize_view_bias_data(view_bias_data, int(q.shape[0]), int(q.shape[1]), int(k.shape[1]),
                                         q.device, q.dtype)
        if norm is not None:
            if softmax_scale is None:
                softmax_scale = 1.0 / math.sqrt(q.shape[-1])
            return SparseTopkIndexerViewBiasFunc.apply(q, k, w, mask, norm["q_view_ids"], norm["s_view_ids"],
                                                       norm["view_bias"], topk, float(softmax_scale), block_k,
                                                       int(merge_blocks))
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
