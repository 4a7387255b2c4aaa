"""Backward of sparse-index attention (gfx950).

Reference: ``SparseIndexFlashAttnFunc.backward`` and ``_sparse_index_flash_attn_backward``
(``easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:3240-3283,2442-2846``):
``dattn_sum`` is cast to q's dtype (``:3244-3245``), gradients are accumulated in fp32 and
returned in the input dtype (``:3247-3282``). Two implementations, neither with float
atomics, so gradients are reproducible:

* ``gw_sparse_attn_bwd_dense``: masked dense passes on the matrix cores, for D = 64 without
  an attn_sum gradient (the reference presets detach the attention mass before the indexer
  loss, ``easyvolcap/official_vggt/layers/dsa_attention.py:4694-4695``) when a query selects
  at least 1 / ``DENSE_MAX_RATIO`` of the keys. A batch element with a position listed twice
  in a row or a non-finite input is reported back by the kernels and the call is redone by
  the CSR path.
* ``gw_sparse_attn_bwd``: gathers over the selected rows, with dK/dV from a key-major
  reduction over the CSR of ``kv_positions``.
"""
from __future__ import annotations

import torch

from .. import _csr, _lib

# "auto": the dense passes when they apply (see above), else the CSR path; "dense" forces
# the dense passes whenever they can run at all, "csr" the CSR path (tests, measurements).
BACKWARD_PATH = "auto"
DENSE_MAX_RATIO = 96
# The dense kernels' 32-bit load offsets bound the token strides and T, S (DENSE_MAX_*): 64
# rows of the transposed operands stay below 2^32 bytes while T (padded to a multiple of 256)
# and S (padded to a multiple of 128) stay below 2^25.
# The grid of at most 65535 query blocks (whole workgroups of 8) bounds T further.
DENSE_MAX_ROW_STRIDE = 1 << 23
DENSE_MAX_LEN = (1 << 25) - 256
DENSE_MAX_T = 65528 * 32
# The path the last call took ("dense" or "csr"), for tests.
last_path = None


def _strides(x: torch.Tensor, layout: str):
    if layout == "bthd":
        return x.stride(0), x.stride(1), x.stride(2)
    return x.stride(0), x.stride(2), x.stride(1)


def _aligned(x: torch.Tensor) -> torch.Tensor:
    if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:-1]) or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def _dense_fits(q, k, v, do, q_layout: str) -> bool:
    """The dense backward's limits: token strides and T, S (32-bit load offsets), T (grid)."""
    t_dim = 2 if q_layout == "bhtd" else 1
    lens = (q.shape[t_dim], k.shape[t_dim])
    return (all(n <= DENSE_MAX_LEN for n in lens) and lens[0] <= DENSE_MAX_T
            and all(_strides(x, q_layout)[1] < DENSE_MAX_ROW_STRIDE for x in (q, k, v, do)))


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
    lib = _lib.load()
    global last_path
    dense_ok = (d == 64 and dattn_sum is None and 0.0 < float(softmax_scale) < float("inf")
                and BACKWARD_PATH != "csr" and _dense_fits(q, k, v, do, q_layout))
    if dense_ok and (BACKWARD_PATH == "dense" or seqlen_k <= DENSE_MAX_RATIO * num_kv):
        ws_bytes = int(lib.gw_sparse_attn_bwd_dense_workspace_size(batch, seqlen_q, seqlen_k, nheads, d, num_kv))
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        route = torch.empty(batch, device=q.device, dtype=torch.int32)
        rc = lib.gw_sparse_attn_bwd_dense(
            _lib.dtype_code(q.dtype),
            q.data_ptr(), _lib.strides3(*_strides(q, q_layout)),
            k.data_ptr(), _lib.strides3(*_strides(k, q_layout)),
            v.data_ptr(), _lib.strides3(*_strides(v, q_layout)),
            kv_positions.data_ptr(), kv_positions.stride(0), kv_positions.stride(1),
            o.data_ptr(), _lib.strides3(*_strides(o, q_layout)),
            do.data_ptr(), _lib.strides3(*_strides(do, q_layout)),
            lse.data_ptr(),
            dq.data_ptr(), _lib.strides3(*_strides(dq, q_layout)),
            dk.data_ptr(), _lib.strides3(*_strides(dk, q_layout)),
            dv.data_ptr(), _lib.strides3(*_strides(dv, q_layout)),
            batch, seqlen_q, seqlen_k, nheads, d, num_kv, float(softmax_scale),
            route.data_ptr(), ws.data_ptr(), ws_bytes,
            _lib.stream_handle(q.device),
        )
        _lib.check(rc, "gw_sparse_attn_bwd_dense")
        del ws
        # Reading the flags waits for the passes; a flagged batch element (a repeated position
        # or a non-finite input) is rare, and then the whole call is redone by the CSR path.
        if not bool(route.any()):
            last_path = "dense"
            return dq, dk, dv
    last_path = "csr"
    csr, csr_bytes = _csr.build(kv_positions, seqlen_k)
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
