"""fp32 CPU restatement of sparse-index attention (forward and backward).

Test infrastructure only (see ``oracle/__init__.py``).

Layout follows the reference's default "bthd": q ``[B,T,H,D]``, k/v ``[B,S,H,D]``,
kv_positions ``[B,T,K]`` int32 shared by all heads.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch


def _scale(head_dim: int, softmax_scale: Optional[float]) -> float:
    # reference: sparse_index_flash_attn.py:2042 (softmax_scale or 1/sqrt(d))
    return float(softmax_scale) if softmax_scale else 1.0 / math.sqrt(head_dim)


def _valid(pos: torch.Tensor, src_len: int) -> torch.Tensor:
    # reference: sparse_index_flash_attn.py:207-209 (pos >= 0 and pos < seqlen_k)
    return (pos >= 0) & (pos < src_len)


def sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    softmax_scale: Optional[float] = None,
    query_chunk: int = 64,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (o fp32 [B,T,H,D], attn_sum fp32 [B,T,K], lse fp32 [B,T,H]).

    Per (b, t, h): p_j = softmax_j(scale * q . k[pos_j]) over valid j, o = sum_j p_j v[pos_j];
    attn_sum[b,t,j] = sum_h p_j. Restates ``_reference_sparse_attn`` (reference
    ``tests/sparse_index_flash_attn_tests.py:47-71``: clamp-gather, masked_fill(-inf),
    softmax, masked_fill(0), sum over heads) which equals ``DSAAttention._sparse_attention``
    (``dsa_attention.py:4731-4753``) when every position is valid. A row with no valid
    position yields o = 0, attn_sum = 0 and lse = -inf (the masked softmax's 0 after
    masked_fill). lse is the natural-log log-sum-exp of the scaled scores
    (``sparse_index_flash_attn.py:225-231``). Chunking over queries leaves per-row
    arithmetic unchanged.
    """
    q = q.float()
    k = k.float()
    v = v.float()
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    topk = kv_positions.shape[-1]
    scale = _scale(head_dim, softmax_scale)
    o = torch.empty((bsz, tgt_len, n_heads, head_dim), dtype=torch.float32)
    attn_sum = torch.empty((bsz, tgt_len, topk), dtype=torch.float32)
    lse = torch.empty((bsz, tgt_len, n_heads), dtype=torch.float32)
    for b in range(bsz):
        for t0 in range(0, tgt_len, query_chunk):
            t1 = min(t0 + query_chunk, tgt_len)
            pos = kv_positions[b, t0:t1].long()
            valid = _valid(pos, src_len)  # [Tc, K]
            safe = torch.where(valid, pos, torch.zeros_like(pos))
            k_sel = k[b][safe]  # [Tc, K, H, D]
            v_sel = v[b][safe]
            s = torch.einsum("thd,tkhd->thk", q[b, t0:t1], k_sel) * scale
            s = s.masked_fill(~valid[:, None, :], float("-inf"))
            row_lse = torch.logsumexp(s, dim=-1)  # [Tc, H]
            p = torch.softmax(s, dim=-1)
            # invalid entries (and so every entry of a row with none valid, whose softmax is
            # nan) get 0; a nan from the scores themselves (an inf or nan in a selected
            # K row) stays, as in the reference's softmax
            p = p.masked_fill(~valid[:, None, :], 0.0)
            o[b, t0:t1] = torch.einsum("thk,tkhd->thd", p, v_sel)
            attn_sum[b, t0:t1] = p.sum(dim=1)
            lse[b, t0:t1] = row_lse
    return o, attn_sum, lse


def sparse_attention_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    do: torch.Tensor,
    dattn: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    query_chunk: int = 64,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dv) fp32 from the reference kernel's backward formulas.

    Restates ``_bwd_preprocess_do_o_dot`` + ``_bwd_sparse_index_kernel`` (reference
    ``sparse_index_flash_attn.py:534-576,579-743``): delta = sum_d o*dO;
    p = exp(scale*q.k - lse); dp = v.dO (+ dattn); ds = (dp - (delta + sum_j dattn*p)) * p;
    dq = scale * sum_j ds k; dk[pos] += scale * ds * q; dv[pos] += p * dO. Invalid
    positions contribute nothing.
    """
    q = q.float()
    k = k.float()
    v = v.float()
    o = o.float()
    do = do.float()
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    scale = _scale(head_dim, softmax_scale)
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    delta = (o * do).sum(-1)  # [B, T, H]
    for b in range(bsz):
        for t0 in range(0, tgt_len, query_chunk):
            t1 = min(t0 + query_chunk, tgt_len)
            pos = kv_positions[b, t0:t1].long()
            valid = _valid(pos, src_len)
            safe = torch.where(valid, pos, torch.zeros_like(pos))
            k_sel = k[b][safe]
            v_sel = v[b][safe]
            qc = q[b, t0:t1]
            s = torch.einsum("thd,tkhd->thk", qc, k_sel) * scale
            p = torch.exp(s - lse[b, t0:t1].unsqueeze(-1))
            p = torch.where(valid[:, None, :], p, torch.zeros_like(p))
            dp = torch.einsum("tkhd,thd->thk", v_sel, do[b, t0:t1])
            total = delta[b, t0:t1].unsqueeze(-1)
            if dattn is not None:
                da = dattn[b, t0:t1].float().unsqueeze(1)  # [Tc, 1, K]
                dp = dp + da
                total = total + (da * p).sum(-1, keepdim=True)
            ds = (dp - total) * p  # [Tc, H, K]
            dq[b, t0:t1] = scale * torch.einsum("thk,tkhd->thd", ds, k_sel)
            dk_c = scale * ds.unsqueeze(-1) * qc.unsqueeze(2)  # [Tc, H, K, D]
            dv_c = p.unsqueeze(-1) * do[b, t0:t1].unsqueeze(2)
            keep = valid.reshape(-1)
            flat_pos = safe.reshape(-1)[keep]
            dk[b].index_add_(0, flat_pos, dk_c.permute(0, 2, 1, 3).reshape(-1, n_heads, head_dim)[keep])
            dv[b].index_add_(0, flat_pos, dv_c.permute(0, 2, 1, 3).reshape(-1, n_heads, head_dim)[keep])
    return dq, dk, dv


def sparse_attention_differentiable(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    softmax_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(o, attn_sum) of the textbook forward as differentiable torch ops on the inputs'
    autograd graph (small shapes only): the forward of ``_reference_sparse_attn``
    (reference ``tests/sparse_index_flash_attn_tests.py:47-71``) with attn_sum = sum of p over
    heads (``sparse_index_flash_attn.py:375-458``)."""
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    scale = _scale(head_dim, softmax_scale)
    pos = kv_positions.long()
    valid = _valid(pos, src_len)
    safe = torch.where(valid, pos, torch.zeros_like(pos))
    outs = []
    sums = []
    for b in range(bsz):
        k_sel = k[b][safe[b]]
        v_sel = v[b][safe[b]]
        s = torch.einsum("thd,tkhd->thk", q[b], k_sel) * scale
        s = s.masked_fill(~valid[b][:, None, :], float("-inf"))
        p = torch.softmax(s, dim=-1).masked_fill(~valid[b][:, None, :], 0.0)
        outs.append(torch.einsum("thk,tkhd->thd", p, v_sel))
        sums.append(p.sum(dim=1))
    return torch.stack(outs), torch.stack(sums)


def sparse_attention_autograd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    do: torch.Tensor,
    dattn: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dv) by autograd through the textbook forward (small shapes only).

    Forward as ``_reference_sparse_attn`` (reference
    ``tests/sparse_index_flash_attn_tests.py:47-71``); the loss is
    sum(o * dO) + sum(attn_sum * dattn). Used to pin ``sparse_attention_bwd``.
    """
    q = q.detach().float().requires_grad_()
    k = k.detach().float().requires_grad_()
    v = v.detach().float().requires_grad_()
    o, attn_sum = sparse_attention_differentiable(q, k, v, kv_positions, softmax_scale)
    loss = (o * do.float()).sum()
    if dattn is not None:
        loss = loss + (attn_sum * dattn.float()).sum()
    loss.backward()
    return q.grad, k.grad, v.grad


def sparse_attention_bwd_keys(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    do: torch.Tensor,
    keys: torch.Tensor,
    softmax_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(dk, dv) fp32 ``[B, len(keys), H, D]`` of the given key rows only, with no dattn.

    Same formulas as ``sparse_attention_bwd`` (reference ``sparse_index_flash_attn.py:
    534-743``) restricted to the (t, j) entries whose position is one of ``keys``: with
    dattn absent, total = delta = sum_d o*dO depends on the query row alone, so a key's
    gradient needs only the rows that select it. Used to check full-size layers where the
    whole oracle backward would take minutes.
    """
    q = q.float()
    k = k.float()
    v = v.float()
    o = o.float()
    do = do.float()
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    scale = _scale(head_dim, softmax_scale)
    keys = keys.long()
    dk = torch.zeros((bsz, keys.numel(), n_heads, head_dim), dtype=torch.float32)
    dv = torch.zeros_like(dk)
    num_kv = kv_positions.shape[-1]
    for b in range(bsz):
        flat = kv_positions[b].reshape(-1).long()
        hit = torch.isin(flat, keys).nonzero().squeeze(1)  # entries that select a key
        t_all, s_all = hit // num_kv, flat[hit]
        for ki, s in enumerate(keys.tolist()):
            t_idx = t_all[s_all == s]  # one entry per (t, j) match
            if t_idx.numel() == 0 or not (0 <= s < src_len):
                continue
            qt = q[b, t_idx]  # [n, H, D]
            dot = do[b, t_idx]
            delta = (o[b, t_idx] * dot).sum(-1)  # [n, H]
            sc = (qt * k[b, s]).sum(-1) * scale
            p = torch.exp(sc - lse[b, t_idx])
            dp = (v[b, s] * dot).sum(-1)
            ds = (dp - delta) * p
            dk[b, ki] = scale * (ds.unsqueeze(-1) * qt).sum(0)
            dv[b, ki] = (p.unsqueeze(-1) * dot).sum(0)
    return dk, dv
