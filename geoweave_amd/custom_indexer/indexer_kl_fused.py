"""Indexer KL training loss on gfx950: the drop-in for the reference module
``easyvolcap/utils/custom_indexer/indexer_kl_fused.py``.

``sparse_indexer_kl_loss(attn_sum, logits, eps=1e-6) -> fp32 scalar`` (reference ``:285-298``):
the mean over the ``B*T`` rows of ``KL(p || softmax(logits))`` with ``p = attn_sum /
(attn_sum.sum(-1) + eps)`` and ``log(p + eps)`` in the entropy term, differentiable w.r.t.
``attn_sum`` and ``logits``. The DSA layer calls it with ``p`` = the attention mass each
query puts on its top-k keys and ``logits`` = the indexer's top-k scores
(``easyvolcap/official_vggt/layers/dsa_attention.py:4688-4715``).

Differences from the reference, all at its edges: it falls back to a torch formula for CPU
tensors and shape mismatches (``:286-295``); here those raise, since this package has no
CPU path. The backward reads ``dL/dloss`` on the device instead of calling ``.item()``
(``:252``), so it does not synchronise the host.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["sparse_indexer_kl_loss", "SparseIndexerKLLossFunc", "sparse_attention_kl_loss"]


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return _lib.GW_DTYPE_FP32
    return _lib.dtype_code(dtype)


def _prepare(attn_sum: torch.Tensor, logits: torch.Tensor):
    if not (torch.is_tensor(attn_sum) and torch.is_tensor(logits)):
        raise TypeError("attn_sum and logits must be tensors")
    if attn_sum.dim() != 3 or tuple(attn_sum.shape) != tuple(logits.shape):
        raise ValueError(
            f"attn_sum {tuple(attn_sum.shape)} and logits {tuple(logits.shape)} must be equal [B, T, K]"
        )
    if not (attn_sum.is_cuda and logits.is_cuda):
        raise ValueError("attn_sum and logits must be GPU tensors")
    # reference: indexer_kl_fused.py:167-172 (contiguous rows, logits cast to attn's dtype)
    attn_sum = attn_sum.contiguous()
    logits = logits.to(attn_sum.dtype).contiguous()
    return attn_sum, logits


def kl_loss_forward(attn_sum: torch.Tensor, logits: torch.Tensor, eps: float) -> torch.Tensor:
    """Per-row losses, fp32 ``[B*T]`` (gw_indexer_kl_fwd on the current stream)."""
    rows = attn_sum.shape[0] * attn_sum.shape[1]
    K = attn_sum.shape[2]
    row_loss = torch.empty(rows, device=attn_sum.device, dtype=torch.float32)
    lib = _lib.load()
    _lib.check(
        lib.gw_indexer_kl_fwd(
            _dtype_code(attn_sum.dtype), attn_sum.data_ptr(), logits.data_ptr(), rows, K, float(eps),
            row_loss.data_ptr(), _lib.stream_handle(attn_sum.device),
        ),
        "gw_indexer_kl_fwd",
    )
    return row_loss


def kl_loss_backward(attn_sum: torch.Tensor, logits: torch.Tensor, grad_out: torch.Tensor, eps: float):
    """(d_attn, d_logits) in the input dtype; ``grad_out`` is dL/dloss on the device."""
    rows = attn_sum.shape[0] * attn_sum.shape[1]
    K = attn_sum.shape[2]
    g = grad_out.detach().reshape(()).to(device=attn_sum.device, dtype=torch.float32).contiguous()
    d_attn = torch.empty_like(attn_sum)
    d_logits = torch.empty_like(logits)
    lib = _lib.load()
    _lib.check(
        lib.gw_indexer_kl_bwd(
            _dtype_code(attn_sum.dtype), attn_sum.data_ptr(), logits.data_ptr(), g.data_ptr(), rows, K,
            float(eps), d_attn.data_ptr(), d_logits.data_ptr(), _lib.stream_handle(attn_sum.device),
        ),
        "gw_indexer_kl_bwd",
    )
    return d_attn, d_logits


class SparseIndexerKLLossFunc(torch.autograd.Function):
    """Autograd wrapper (reference ``_SparseIndexerKLLossFunc``, ``indexer_kl_fused.py:164-282``)."""

    @staticmethod
    def forward(ctx, attn_sum: torch.Tensor, logits: torch.Tensor, eps: float):
        a, z = _prepare(attn_sum, logits)
        row_loss = kl_loss_forward(a, z, eps)
        ctx.save_for_backward(a, z)
        ctx.eps = float(eps)
        ctx.logits_dtype = logits.dtype
        return row_loss.mean()

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        a, z = ctx.saved_tensors
        d_attn, d_logits = kl_loss_backward(a, z, grad_out, ctx.eps)
        return d_attn, d_logits.to(ctx.logits_dtype), None


def sparse_indexer_kl_loss(attn_sum: torch.Tensor, logits: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Mean KL(p || softmax(logits)) over rows (reference ``indexer_kl_fused.py:285-298``)."""
    if torch.is_tensor(attn_sum) and attn_sum.numel() == 0 and attn_sum.dim() == 3:
        # reference: indexer_kl_fused.py:296-297
        return attn_sum.new_zeros(())
    return SparseIndexerKLLossFunc.apply(attn_sum, logits, float(eps))


class _AttnWithKLRows(torch.autograd.Function):
    """Sparse attention forward that also writes the KL row losses (gw_sparse_attn_fwd_kl);
    the backward is the attention's own, with dattn_sum from the KL node below."""

    @staticmethod
    def forward(ctx, q, k, v, kv_positions, logits, eps, softmax_scale):
        from ..custom_flash_attn.sparse_index_flash_attn import _flash_attn_forward

        # attn_sum without a gradient (the loss on a detached mass) brings None, not zeros
        ctx.set_materialize_grads(False)
        if kv_positions.stride(-1) != 1:
            kv_positions = kv_positions.contiguous()
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        B, T = kv_positions.shape[0], kv_positions.shape[1]
        row_loss = torch.empty(B * T, device=q.device, dtype=torch.float32)
        o, attn_sum, lse, ctx.softmax_scale = _flash_attn_forward(
            q, k, v, kv_positions, softmax_scale=softmax_scale, return_attn=True, q_layout="bthd",
            kl_logits=logits, kl_eps=eps, kl_row_loss=row_loss,
        )
        ctx.save_for_backward(q, k, v, kv_positions, o, lse)
        ctx.mark_non_differentiable(row_loss)
        return o, attn_sum, row_loss

    @staticmethod
    def backward(ctx, do, dattn_sum, _d_row_loss):
        from ..custom_flash_attn.sparse_index_flash_attn import _flash_attn_backward

        q, k, v, kv_positions, o, lse = ctx.saved_tensors
        dq, dk, dv = _flash_attn_backward(do, q, k, v, kv_positions, o, lse, dattn_sum, ctx.softmax_scale, "bthd")
        return dq, dk, dv, None, None, None, None


class _KLFromRowLosses(torch.autograd.Function):
    """The mean of row losses computed in the attention epilogue; backward as
    SparseIndexerKLLossFunc (gw_indexer_kl_bwd on attn_sum and the fp32 logits)."""

    @staticmethod
    def forward(ctx, attn_sum, logits, row_loss, eps):
        a, z = _prepare(attn_sum, logits)
        ctx.save_for_backward(a, z)
        ctx.eps = float(eps)
        ctx.logits_dtype = logits.dtype
        return row_loss.mean()

    @staticmethod
    def backward(ctx, grad_out):
        a, z = ctx.saved_tensors
        d_attn, d_logits = kl_loss_backward(a, z, grad_out, ctx.eps)
        return (d_attn if ctx.needs_input_grad[0] else None), d_logits.to(ctx.logits_dtype), None, None


def sparse_attention_kl_loss(q, k, v, kv_positions, logits, eps: float = 1e-6, softmax_scale=None,
                             detach_input: bool = False):
    """``(o, attn_sum, loss)``: ``sparse_index_flash_attn_func(q, k, v, kv_positions)``
    followed by ``sparse_indexer_kl_loss(attn_sum, logits, eps)`` (reference
    ``dsa_attention.py:5395-5411`` with the attention mass as p), with the loss's forward
    fused into the attention's attn_sum epilogue: attn_sum is not read back for the loss.
    Same values and gradients as the two calls (the fused sums run in another order);
    ``logits`` is the indexer's ``topk_scores`` aligned with ``kv_positions``.
    ``detach_input``: the loss sees the attention mass detached (the reference's indexer
    option of that name, on in its presets, ``dsa_attention.py:4694-4695``), so the loss
    trains the indexer only and brings no gradient into q, k, v."""
    if logits.shape != kv_positions.shape:
        raise ValueError(f"logits {tuple(logits.shape)} must match kv_positions {tuple(kv_positions.shape)}")
    o, attn_sum, row_loss = _AttnWithKLRows.apply(q, k, v, kv_positions, logits, float(eps), softmax_scale)
    p = attn_sum.detach() if detach_input else attn_sum
    return o, attn_sum, _KLFromRowLosses.apply(p, logits, row_loss, float(eps))
