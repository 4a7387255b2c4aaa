"""fp64 CPU restatement of the indexer KL training loss and its backward.

Test infrastructure only (see ``oracle/__init__.py``).

Reference: ``sparse_indexer_kl_loss`` (``easyvolcap/utils/custom_indexer/indexer_kl_fused.py:
158-298``; row kernels ``:8-155``) and the torch loss it replaces
(``easyvolcap/official_vggt/layers/dsa_attention.py:4713-4715``).
"""
from __future__ import annotations

from typing import Tuple

import torch


def _rows(attn_sum: torch.Tensor, logits: torch.Tensor):
    if attn_sum.shape != logits.shape or attn_sum.dim() != 3:
        raise ValueError("attn_sum and logits must both be [B, T, K]")
    a = attn_sum.detach().double().reshape(-1, attn_sum.shape[-1])
    z = logits.detach().to(attn_sum.dtype).double().reshape(-1, logits.shape[-1])
    return a, z


def kl_row_losses(attn_sum: torch.Tensor, logits: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Per-row loss, fp64 ``[B*T]``.

    ``p = attn / (sum attn + eps)`` (``indexer_kl_fused.py:76-86``), ``log_q = z - max z -
    log sum exp(z - max z)`` (``:74-85``), ``row = sum p (log(p + eps) - log_q)`` (``:86-91``).
    Logits are first cast to ``attn_sum``'s dtype (``:171-172``).
    """
    a, z = _rows(attn_sum, logits)
    p = a / (a.sum(-1, keepdim=True) + eps)
    zm = z.max(-1, keepdim=True).values
    log_q = z - zm - torch.log(torch.exp(z - zm).sum(-1, keepdim=True))
    return (p * (torch.log(p + eps) - log_q)).sum(-1)


def kl_loss(attn_sum: torch.Tensor, logits: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Mean of the row losses (``indexer_kl_fused.py:232``), fp64 scalar."""
    return kl_row_losses(attn_sum, logits, eps).mean()


def kl_loss_bwd(
    attn_sum: torch.Tensor, logits: torch.Tensor, grad_out: float, eps: float = 1e-6
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(d_attn, d_logits), fp64 ``[B, T, K]``: the reference's explicit gradient
    (``indexer_kl_fused.py:123-155``, ``:252``):
    ``gs = grad_out / rows``; ``g = log(p + eps) - log_q + p / (p + eps)``;
    ``gbar = sum p g``; ``d_attn = (g - gbar) gs / (sum attn + eps)``;
    ``d_logits = (softmax(z) - p) gs``.

    ``d_attn`` is the exact derivative. ``d_logits`` is the reference's: the exact one is
    ``(softmax(z) sum(p) - p) gs`` with ``sum(p) = S / (S + eps)``, so the two differ by
    ``softmax(z) eps / (S + eps) gs`` (zero for eps = 0; relative 1e-6 for the layer's
    pre-normalised p, ``dsa_attention.py:5410``).
    """
    a, z = _rows(attn_sum, logits)
    rows = a.shape[0]
    gs = float(grad_out) / max(1, rows)
    denom = a.sum(-1, keepdim=True) + eps
    p = a / denom
    zm = z.max(-1, keepdim=True).values
    log_q = z - zm - torch.log(torch.exp(z - zm).sum(-1, keepdim=True))
    g = torch.log(p + eps) - log_q + p / (p + eps)
    gbar = (p * g).sum(-1, keepdim=True)
    d_attn = (g - gbar) * gs / denom
    d_logits = (torch.exp(log_q) - p) * gs
    return d_attn.reshape(attn_sum.shape), d_logits.reshape(logits.shape)


def kl_loss_autograd(attn_sum: torch.Tensor, logits: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """The reference's torch formula as differentiable ops in the inputs' dtype
    (``indexer_kl_fused.py:158-161``): ``p = attn / (sum attn + eps)``,
    ``mean((p * (log(p + eps) - log_softmax(logits))).sum(-1))``. Its logits gradient is the
    exact one (see ``kl_loss_bwd`` for the fused kernel's)."""
    p = attn_sum / (attn_sum.sum(dim=-1, keepdim=True) + eps)
    log_q = torch.log_softmax(logits, dim=-1)
    return (p * (torch.log(p + eps) - log_q)).sum(dim=-1).mean()
