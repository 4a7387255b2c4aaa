"""Key-major (CSR) transpose of a ``[B, T, K]`` position table on the GPU.

Both backward passes of a sparse global-attention layer reduce gradients per selected key:
the attention's dK/dV over ``kv_positions`` and the indexer's dK/dW over ``topk_indices``,
which are the same table in a layer (reference ``dsa_attention.py:5288-5291`` converts
the indexer's indices into ``kv_positions``). The CSR is built by ``gw_kv_csr_build`` and
kept for the most recent table, so the second backward of a layer reuses the first one's
build. The single entry is keyed on the table's storage, shape, strides and version
counter (so an in-place change invalidates it) and holds a reference to the table, so
the storage cannot be recycled under the key while the entry lives. The next build
replaces the entry; ``clear_cache()`` drops it (and its buffer) at once.
"""
from __future__ import annotations

import threading
from typing import Tuple

import torch

from . import _lib

_lock = threading.Lock()
_cache: list = []  # [(key, table, csr tensor)], most recent last
_CACHE_SIZE = 1


def _key(pos: torch.Tensor, src_len: int) -> Tuple:
    return (pos.device, pos.data_ptr(), tuple(pos.shape), tuple(pos.stride()), pos._version, int(src_len))


def build(pos: torch.Tensor, src_len: int, cache: bool = True) -> Tuple[torch.Tensor, int]:
    """(csr buffer, size in bytes) for an int32 ``[B, T, K]`` table with unit last stride."""
    if pos.dtype != torch.int32 or pos.dim() != 3:
        raise TypeError("position table must be int32 [B, T, K]")
    if pos.stride(-1) != 1:
        pos = pos.contiguous()
    key = _key(pos, src_len)
    if cache:
        with _lock:
            for k, _, csr in _cache:
                if k == key:
                    return csr, csr.numel()
    bsz, tgt_len, num_kv = pos.shape
    lib = _lib.load()
    nbytes = int(lib.gw_kv_csr_size(bsz, tgt_len, src_len, num_kv))
    csr = torch.empty(nbytes, device=pos.device, dtype=torch.uint8)
    # the sort's ping-pong buffers are transient: torch's caching allocator takes the block
    # back when this tensor dies (after the queued kernels, on this stream), so only the
    # table itself stays cached
    ws_bytes = int(lib.gw_kv_csr_build_workspace_size(bsz, tgt_len, src_len, num_kv))
    ws = torch.empty(ws_bytes, device=pos.device, dtype=torch.uint8)
    rc = lib.gw_kv_csr_build(
        pos.data_ptr(), pos.stride(0), pos.stride(1), bsz, tgt_len, src_len, num_kv,
        csr.data_ptr(), nbytes, ws.data_ptr(), ws_bytes, _lib.stream_handle(pos.device),
    )
    _lib.check(rc, "gw_kv_csr_build")
    del ws
    if cache:
        with _lock:
            _cache.append((key, pos, csr))
            del _cache[:-_CACHE_SIZE]
    return csr, nbytes


def clear_cache() -> None:
    with _lock:
        _cache.clear()
