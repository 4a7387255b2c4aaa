"""Backward of sparse-index attention through ``gw_sparse_attn_bwd`` (gfx950).

Reference: ``SparseIndexFlashAttnFunc.backward`` and ``_sparse_index_flash_attn_backward``
(``easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:3240-3283,2442-2846``):
``dattn_sum`` is cast to q's dtype (``:3244-3245``), gradients are accumulated in fp32 and
returned in the input dtype (``:3247-3282``). Here dK/dV come from a key-major reduction
over the CSR of ``kv_positions`` instead of fp32 atomics, so they are reproducible.
"""
from __future__ import annotations

import torch

from .. import _csr, _lib


def _strides(x: torch.Tensor, layout: str):
    if layout == "bthd":
        return x.stride(0), x.stride(1), x.stride(2)
    return x.stride(0), x.stride(2), x.stride(1)


def _aligned(x: torch.Tensor) -> torch.Tensor:
    if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:-1]) or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def sparse_attn_backward(do, q, k, v, kv_positions, o, lse, dattn_sum, softmax_scale, q_layout):
    """(dq, dk, dv) in the dtype and layout of (q, k, v)."""
    if q_layout == "bthd":
        batch, seqlen_q, nheads, d = q.shape
        seqlen_k = k.shape[1]
    else:
        batch, nheads, seqlen_q, d = q.shape
        seqlen_k = k.shape[2]
    num_kv = kv_positions.shape[-1]
    if do is None:
        do = torch.zeros_like(o)
    do = _aligned(do.to(q.dtype))
    dq = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    dk = torch.empty(k.shape, device=k.device, dtype=k.dtype)
    dv = torch.empty(v.shape, device=v.device, dtype=v.dtype)
    if batch == 0 or seqlen_q == 0 or seqlen_k == 0 or num_kv == 0:
        dq.zero_()
        dk.zero_()
        dv.zero_()
        return dq, dk, dv
    if dattn_sum is not None:
        dattn_sum = dattn_sum.to(q.dtype).contiguous()
    if kv_positions.stride(-1) != 1:
        kv_positions = kv_positions.contiguous()
    csr, csr_bytes = _csr.build(kv_positions, seqlen_k)
    lib = _lib.load()
    ws_bytes = int(lib.gw_sparse_attn_bwd_workspace_size(batch, seqlen_q, seqlen_k, nheads, d, num_kv))
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    rc = lib.gw_sparse_attn_bwd(
        _lib.dtype_code(q.dtype),
        q.data_ptr(), _lib.strides3(*_strides(q, q_layout)),
        k.data_ptr(), _lib.strides3(*_strides(k, q_layout)),
        v.data_ptr(), _lib.strides3(*_strides(v, q_layout)),
        kv_positions.data_ptr(), kv_positions.stride(0), kv_positions.stride(1),
        o.data_ptr(), _lib.strides3(*_strides(o, q_layout)),
        do.data_ptr(), _lib.strides3(*_strides(do, q_layout)),
        lse.data_ptr(), _lib.ptr(dattn_sum),
        dq.data_ptr(), _lib.strides3(*_strides(dq, q_layout)),
        dk.data_ptr(), _lib.strides3(*_strides(dk, q_layout)),
        dv.data_ptr(), _lib.strides3(*_strides(dv, q_layout)),
        batch, seqlen_q, seqlen_k, nheads, d, num_kv, float(softmax_scale),
        csr.data_ptr(), csr_bytes, ws.data_ptr(), ws_bytes,
        _lib.stream_handle(q.device),
    )
    _lib.check(rc, "gw_sparse_attn_bwd")
    return dq, dk, dv
