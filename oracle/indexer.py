"""fp32 CPU restatement of the lightning-indexer score, exact top-k and its backward.

Test infrastructure only (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch


def _default_scale(head_dim: int, softmax_scale: Optional[float]) -> float:
    # reference: sparse_topk_indexer.py:2063-2064 (softmax_scale None -> 1/sqrt(D))
    return float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(head_dim)


def indexer_scores(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    mask: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    key_chunk: int = 4096,
    query_chunk: int = 2048,
    view_bias: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
) -> torch.Tensor:
    """score[b,t,s] = sum_h w[b,s,h] * relu(scale * <q[b,t,h], k[b,s,h]>) (+ mask[b,t,s])
    (+ view_bias[b, q_view[b,t], s_view[b,s]]).

    Restates ``LightningIndexer._compute_scores`` / ``_compute_score_chunk``
    (reference ``easyvolcap/official_vggt/layers/indexer.py:383-466``) with every head in
    one head chunk (``score_head_chunk_size`` 0 or = n_heads, ``indexer.py:108-113``):
    ``einsum('bthd,bshd->bths') * scale -> relu -> * w[:, None] -> sum(dim=2)``, then the
    additive mask (``indexer.py:412-415``). Everything is fp32 (the torch backend's
    ``score_dtype='float32'``, ``geoweave/inference.py:58``). Chunking over keys is the
    reference's own ``score_key_chunk_size`` loop; chunking over queries leaves per-row
    arithmetic unchanged. ``view_bias`` = (q_view_ids [B,T], s_view_ids [B,S], table
    [B,Vq,Vs]): the soft view-bias term, added after the mask (``_compute_score_chunk``,
    ``indexer.py:460-465``; ``sparse_topk_indexer.py:935-951``).
    """
    q = q.float()
    k = k.float()
    w = w.float()
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    scale = torch.tensor(_default_scale(head_dim, softmax_scale), dtype=torch.float32)
    w_by_head = w.permute(0, 2, 1)  # [B, Hi, S]
    out = torch.empty((bsz, tgt_len, src_len), dtype=torch.float32)
    for t0 in range(0, tgt_len, query_chunk):
        t1 = min(t0 + query_chunk, tgt_len)
        q_c = q[:, t0:t1]
        for s0 in range(0, src_len, key_chunk):
            s1 = min(s0 + key_chunk, src_len)
            hs = torch.einsum("bthd,bshd->bths", q_c, k[:, s0:s1]) * scale
            hs = torch.relu(hs)
            hs = hs * w_by_head[:, :, s0:s1].unsqueeze(1)
            out[:, t0:t1, s0:s1] = hs.sum(dim=2, dtype=torch.float32)
    if mask is not None and mask.numel() > 0:
        out = out + mask.float()
    if view_bias is not None:
        out = out + view_bias_term(*view_bias)
    return out


def view_bias_term(q_view_ids: torch.Tensor, s_view_ids: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """fp32 ``[B,T,S]``: ``table[b, q_view_ids[b,t], s_view_ids[b,s]]`` (reference
    ``LightningIndexer._compute_view_bias_chunk``, ``indexer.py:509-519``, over the whole key
    range; ids ``[B,T]``/``[B,S]``, table ``[B,Vq,Vs]``)."""
    qv = q_view_ids.long()
    sv = s_view_ids.long()
    tab = table.float()
    bidx = torch.arange(tab.shape[0]).view(-1, 1, 1)
    return tab[bidx, qv.unsqueeze(-1), sv.unsqueeze(1)]


def view_bias_grad(indices: torch.Tensor, grad_scores: torch.Tensor, q_view_ids: torch.Tensor,
                   s_view_ids: torch.Tensor, table_shape) -> torch.Tensor:
    """fp32 gradient of the table from the selected scores' gradient: for every selected
    (b, t, j), ``grad[b, q_view[b,t], s_view[b, indices[b,t,j]]] += grad_scores[b,t,j]``.
    Restates ``_scatter_view_bias_grad`` (reference ``sparse_topk_indexer.py:898-932``: flat
    index ``b*Vq*Vs + q_view*Vs + s_view``, fp32 ``scatter_add_``)."""
    bsz, n_q, n_s = table_shape
    idx = indices.long()
    sv_sel = torch.gather(s_view_ids.long(), 1, idx.reshape(bsz, -1)).view_as(idx)  # [B,T,K]
    lin = (torch.arange(bsz).view(-1, 1, 1) * (n_q * n_s) + q_view_ids.long().unsqueeze(-1) * n_s + sv_sel)
    out = torch.zeros(bsz * n_q * n_s, dtype=torch.float32)
    out.scatter_add_(0, lin.reshape(-1), grad_scores.float().reshape(-1))
    return out.view(bsz, n_q, n_s)


def indexer_topk(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    mask: Optional[torch.Tensor],
    topk: int,
    softmax_scale: Optional[float] = None,
    query_chunk: int = 1024,
    view_bias: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(indices int32 [B,T,K], scores fp32 [B,T,K]) of the K largest scores per row.

    Restates ``LightningIndexer.select_topk_projected``'s torch branch (reference
    ``indexer.py:546,600-603``): ``topk = min(topk, S)``, ``scores.topk(topk, dim=-1,
    sorted=False)``, ``scores.gather(-1, idx)``. The caller converts indices to int32
    (``dsa_attention.py:5288``). Order within a row is unspecified.
    """
    bsz, tgt_len = q.shape[:2]
    src_len = k.shape[1]
    kk = min(int(topk), int(src_len))
    idx = torch.empty((bsz, tgt_len, kk), dtype=torch.int32)
    val = torch.empty((bsz, tgt_len, kk), dtype=torch.float32)
    for t0 in range(0, tgt_len, query_chunk):
        t1 = min(t0 + query_chunk, tgt_len)
        m = None if mask is None or mask.numel() == 0 else mask[:, t0:t1]
        vb = None if view_bias is None else (view_bias[0][:, t0:t1], view_bias[1], view_bias[2])
        sc = indexer_scores(q[:, t0:t1], k, w, m, softmax_scale, view_bias=vb)
        v, i = sc.topk(kk, dim=-1, sorted=False)
        idx[:, t0:t1] = i.to(torch.int32)
        val[:, t0:t1] = v
    return idx, val


def selected_scores(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    indices: torch.Tensor,
    softmax_scale: Optional[float] = None,
) -> torch.Tensor:
    """fp32 score of each selected (t, indices[t, j]) pair, same formula as
    ``indexer_scores`` evaluated only at the selected keys (reference
    ``sparse_topk_indexer.py:1924-1933``: z = scale * q . k_idx; relu; * w_idx; sum over h).
    Invalid (negative) indices give NaN so they cannot pass a comparison silently."""
    q = q.float()
    k = k.float()
    w = w.float()
    head_dim = q.shape[-1]
    scale = _default_scale(head_dim, softmax_scale)
    idx = indices.long()
    valid = idx >= 0
    safe = idx.clamp(min=0)
    bsz = q.shape[0]
    out = torch.empty(idx.shape, dtype=torch.float32)
    for b in range(bsz):
        k_sel = k[b][safe[b]]  # [T, K, Hi, Di]
        w_sel = w[b][safe[b]]  # [T, K, Hi]
        z = torch.einsum("thd,tkhd->tkh", q[b], k_sel) * scale
        out[b] = (torch.relu(z) * w_sel).sum(dim=-1)
    out[~valid] = float("nan")
    return out


def indexer_topk_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    indices: torch.Tensor,
    grad_scores: torch.Tensor,
    softmax_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dw) fp32 for score = sum_h w_idx,h * relu(scale * q_h . k_idx,h).

    Restates ``_indexer_topk_bwd_kernel`` (reference
    ``easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:1847-1944``):
    z = scale * q.k_idx; f = g * w_idx * [z > 0] * scale; dq = sum_j f * k_idx;
    dk[idx] += f * q; dw[idx] += g * relu(z). Accumulation is fp32 (``:757-776``).
    """
    q = q.float()
    k = k.float()
    w = w.float()
    g = grad_scores.float()
    bsz, tgt_len, n_heads, head_dim = q.shape
    scale = _default_scale(head_dim, softmax_scale)
    idx = indices.long()
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dw = torch.zeros_like(w)
    for b in range(bsz):
        k_sel = k[b][idx[b]]  # [T, K, H, D]
        w_sel = w[b][idx[b]]  # [T, K, H]
        z = torch.einsum("thd,tkhd->tkh", q[b], k_sel) * scale
        pos = (z > 0).float()
        f = g[b].unsqueeze(-1) * w_sel * pos * scale  # [T, K, H]
        dq[b] = torch.einsum("tkh,tkhd->thd", f, k_sel)
        dk_contrib = f.unsqueeze(-1) * q[b].unsqueeze(1)  # [T, K, H, D]
        dk[b].index_add_(0, idx[b].reshape(-1), dk_contrib.reshape(-1, n_heads, head_dim))
        dw_contrib = g[b].unsqueeze(-1) * torch.relu(z)  # [T, K, H]
        dw[b].index_add_(0, idx[b].reshape(-1), dw_contrib.reshape(-1, n_heads))
    return dq, dk, dw


def indexer_topk_bwd_keys(
    q: torch.Tensor,
    k: torch.Tensor,
    w: torch.Tensor,
    indices: torch.Tensor,
    grad_scores: torch.Tensor,
    keys: torch.Tensor,
    softmax_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(dk, dw) fp32 of the given key rows only: the formulas of ``indexer_topk_bwd``
    (reference ``sparse_topk_indexer.py:1847-1944``) restricted to the (t, j) entries that
    select one of ``keys``. Used to check full-size layers."""
    q = q.float()
    k = k.float()
    w = w.float()
    g = grad_scores.float()
    bsz, tgt_len, n_heads, head_dim = q.shape
    scale = _default_scale(head_dim, softmax_scale)
    keys = keys.long()
    dk = torch.zeros((bsz, keys.numel(), n_heads, head_dim), dtype=torch.float32)
    dw = torch.zeros((bsz, keys.numel(), n_heads), dtype=torch.float32)
    num_topk = indices.shape[-1]
    for b in range(bsz):
        flat = indices[b].reshape(-1).long()
        hit = torch.isin(flat, keys).nonzero().squeeze(1)
        t_all, j_all, s_all = hit // num_topk, hit % num_topk, flat[hit]
        for ki, s in enumerate(keys.tolist()):
            m = s_all == s
            t_idx, j_idx = t_all[m], j_all[m]
            if t_idx.numel() == 0:
                continue
            qt = q[b, t_idx]  # [n, H, D]
            gg = g[b, t_idx, j_idx].unsqueeze(-1)  # [n, 1]
            z = (qt * k[b, s]).sum(-1) * scale  # [n, H]
            f = gg * w[b, s] * (z > 0).float() * scale
            dk[b, ki] = (f.unsqueeze(-1) * qt).sum(0)
            dw[b, ki] = (gg * torch.relu(z)).sum(0)
    return dk, dw
