"""Backward of the indexer top-k scores (gfx950).

Reference: ``SparseTopkIndexerFunc.backward`` -> ``_backward_selected_topk_qkw`` ->
``_indexer_topk_bwd_kernel`` (``easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:
2091-2106,757-895,1847-1944``): fp32 accumulation, results cast to the input dtypes.
Two implementations, neither with float atomics, so gradients are reproducible:

* ``gw_indexer_topk_bwd_dense``: masked dense passes on the matrix cores (bf16, Di = 64,
  S <= 65536, k <= 2048) when a query selects at least 1 / ``DENSE_MAX_RATIO`` of the keys.
  A batch element with a position listed twice in a row or a non-finite input is reported
  back by the kernels and the call is redone by the CSR path.
* ``gw_indexer_topk_bwd``: gathers over the selected rows, with dK and dW from a key-major
  reduction over the CSR of ``topk_indices`` (shared with the attention backward of the same
  layer).
"""
from __future__ import annotations

import torch

from .. import _csr, _lib

# "auto": the dense passes when they apply (see above), else the CSR path; "dense" forces
# the dense passes whenever they can run at all, "csr" the CSR path (tests, measurements).
BACKWARD_PATH = "auto"
DENSE_MAX_RATIO = 96
DENSE_MAX_S = 65536
DENSE_MAX_K = 2048
DENSE_MAX_T = (1 << 22) - 32
# The path the last call took ("dense" or "csr"), for tests.
last_path = None


def _aligned(x: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned start (the kernels' vector loads)."""
    if not x.is_contiguous() or x.data_ptr() % 16:
        x = x.contiguous() if not x.is_contiguous() else x.clone()
    return x


def _dense_applies(q, num_topk, src_len, softmax_scale) -> bool:
    n_heads, head_dim = q.shape[2], q.shape[3]
    return (BACKWARD_PATH != "csr" and q.dtype == torch.bfloat16 and head_dim == 64
            and n_heads in (1, 2, 4, 8) and src_len <= DENSE_MAX_S and num_topk <= DENSE_MAX_K
            and q.shape[1] <= DENSE_MAX_T and 0.0 < float(softmax_scale) < float("inf")
            and (BACKWARD_PATH == "dense" or src_len <= DENSE_MAX_RATIO * num_topk))


def indexer_topk_backward(q, k, w, topk_indices, grad_scores, softmax_scale):
    from .sparse_topk_indexer import KERNEL_HEAD_DIM, kernel_heads, pad_head_dim, pad_heads

    d = q.shape[-1]
    if d < KERNEL_HEAD_DIM:
        dq, dk, dw = indexer_topk_backward(pad_head_dim(q), pad_head_dim(k), w, topk_indices, grad_scores,
                                           softmax_scale)
        return dq[..., :d].contiguous(), dk[..., :d].contiguous(), dw
    h = q.shape[2]
    hp = kernel_heads(h, q.dtype)
    if hp is not None and hp != h:
        dq, dk, dw = indexer_topk_backward(pad_heads(q, hp), pad_heads(k, hp), pad_heads(w, hp), topk_indices,
                                           grad_scores, softmax_scale)
        return dq[:, :, :h].contiguous(), dk[:, :, :h].contiguous(), dw[:, :, :h].contiguous()
    global last_path
    bsz, tgt_len, n_heads, head_dim = q.shape
    src_len = k.shape[1]
    num_topk = topk_indices.shape[-1]
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dw = torch.empty_like(w, memory_format=torch.contiguous_format)
    if bsz == 0 or tgt_len == 0 or src_len == 0 or num_topk == 0:
        return dq.zero_(), dk.zero_(), dw.zero_()
    q, k, w = (_aligned(x) for x in (q, k, w))
    grad_scores = _aligned(grad_scores.to(q.dtype))
    topk_indices = _aligned(topk_indices)
    lib = _lib.load()
    if _dense_applies(q, num_topk, src_len, softmax_scale):
        ws_bytes = int(lib.gw_indexer_topk_bwd_dense_workspace_size(bsz, tgt_len, src_len, n_heads, head_dim,
                                                                     num_topk))
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        route = torch.empty(bsz, device=q.device, dtype=torch.int32)
        rc = lib.gw_indexer_topk_bwd_dense(
            _lib.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), w.data_ptr(),
            topk_indices.data_ptr(), grad_scores.data_ptr(), dq.data_ptr(), dk.data_ptr(), dw.data_ptr(),
            bsz, tgt_len, src_len, n_heads, head_dim, num_topk, float(softmax_scale),
            route.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_handle(q.device),
        )
        _lib.check(rc, "gw_indexer_topk_bwd_dense")
        del ws
        # Reading the flags waits for the passes; a flagged batch element (a repeated position
        # or a non-finite input) is rare, and then the whole call is redone by the CSR path.
        if not bool(route.any()):
            last_path = "dense"
            return dq, dk, dw
    last_path = "csr"
    csr, csr_bytes = _csr.build(topk_indices, src_len)
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
