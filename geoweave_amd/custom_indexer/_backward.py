"""Backward of the indexer top-k scores through ``gw_indexer_topk_bwd`` (gfx950).

Reference: ``SparseTopkIndexerFunc.backward`` -> ``_backward_selected_topk_qkw`` ->
``_indexer_topk_bwd_kernel`` (``easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:
2091-2106,757-895,1847-1944``): fp32 accumulation, results cast to the input dtypes.
dK and dW come from a key-major reduction over the CSR of ``topk_indices`` (shared with
the attention backward of the same layer) instead of fp32 atomics.
"""
from __future__ import annotations

import torch

from .. import _csr, _lib


def indexer_topk_backward(q, k, w, topk_indices, grad_scores, softmax_scale):
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    num_topk = topk_indices.shape[-1]
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dw = torch.empty_like(w, memory_format=torch.contiguous_format)
    if bsz == 0 or tgt_len == 0 or src_len == 0 or num_topk == 0:
        return dq.zero_(), dk.zero_(), dw.zero_()
    grad_scores = grad_scores.to(q.dtype).contiguous()
    topk_indices = topk_indices.contiguous()
    csr, csr_bytes = _csr.build(topk_indices, src_len)
    lib = _lib.load()
    ws_bytes = int(lib.gw_indexer_topk_bwd_workspace_size(bsz, tgt_len, src_len, n_heads, head_dim, num_topk))
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    rc = lib.gw_indexer_topk_bwd(
        _lib.dtype_code(q.dtype, allow_fp32=True), q.data_ptr(), k.data_ptr(), w.data_ptr(),
        topk_indices.data_ptr(), grad_scores.data_ptr(), dq.data_ptr(), dk.data_ptr(), dw.data_ptr(),
        bsz, tgt_len, src_len, n_heads, head_dim, num_topk, float(softmax_scale),
        csr.data_ptr(), csr_bytes, ws.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
    )
    _lib.check(rc, "gw_indexer_topk_bwd")
    return dq, dk, dw
