"""ctypes binding of libgeoweave_hip.so (the C ABI declared in include/geoweave_hip.h).

The library is loaded after torch so that both share torch's HIP runtime. There is no
fallback: if the library is missing or a call fails, a RuntimeError says why.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional, Sequence

import torch

LIB_PATH = Path(__file__).resolve().with_name("libgeoweave_hip.so")

GW_OK = 0
GW_DTYPE_BF16 = 0
GW_DTYPE_FP16 = 1
GW_DTYPE_FP32 = 2

_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
_sz = ctypes.c_size_t

# name -> (restype, argtypes). Kept in the order of include/geoweave_hip.h.
_SIGNATURES = {
    "gw_last_error": (ctypes.c_char_p, []),
    "gw_abi_version": (ctypes.c_int, []),
    "gw_sparse_attn_fwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, ctypes.c_int]),
    "gw_sparse_attn_fwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64, _i64, _p, _i64p, _p, _p,
         _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, _sz, _p],
    ),
    "gw_indexer_topk_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "gw_indexer_topk_fwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
         ctypes.c_int, _p, _p, _p, _sz, _p],
    ),
    "gw_indexer_topk_fwd_view_bias": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         ctypes.c_float, ctypes.c_int, _p, _p, _p, _sz, _p],
    ),
    "gw_kv_csr_size": (_sz, [_i64, _i64, _i64, _i64]),
    "gw_kv_csr_build_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "gw_kv_csr_build": (ctypes.c_int, [_p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _sz, _p, _sz, _p]),
    "gw_sparse_attn_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "gw_sparse_attn_bwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64, _i64, _p, _i64p, _p, _i64p,
         _p, _p, _p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64, _i64,
         ctypes.c_float, _p, _sz, _p, _sz, _p],
    ),
    "gw_indexer_topk_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "gw_indexer_topk_bwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
         ctypes.c_float, _p, _sz, _p, _sz, _p],
    ),
    "gw_indexer_topk_bwd_dense_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "gw_indexer_topk_bwd_dense": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
         ctypes.c_float, _p, _p, _sz, _p],
    ),
    "gw_indexer_view_bias_bwd_rows": (
        ctypes.c_int, [ctypes.c_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p],
    ),
    "gw_indexer_kl_fwd": (ctypes.c_int, [ctypes.c_int, _p, _p, _i64, _i64, ctypes.c_float, _p, _p]),
    "gw_indexer_kl_bwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _i64, _i64, ctypes.c_float, _p, _p, _p],
    ),
    "gw_dsa_glue_fwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _p, _p, _p, _p, _p, _p, ctypes.c_float, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p],
    ),
    "gw_dsa_glue_bwd_workspace_size": (_sz, [_i64, _i64, _i64]),
    "gw_dsa_glue_bwd": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _p, _p, _p, _p, _p, _p, ctypes.c_float, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p,
         _p, _sz, _p],
    ),
    "gw_sparse_attn_fwd_kl": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64, _i64, _p, _i64p, _p, _p,
         _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, ctypes.c_int, _i64, _i64,
         ctypes.c_float, _p, _p, _sz, _p],
    ),
    "gw_source_downsample_pool": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, ctypes.c_int, _p, _p, _p],
    ),
    "gw_source_downsample_expand": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, ctypes.c_int, _i64, _i64,
         _p, _i64, _p, _p],
    ),
    "gw_source_downsample_rerank": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
         ctypes.c_float, _p, _p, _p],
    ),
    "gw_source_downsample_subcell_top1": (
        ctypes.c_int,
        [ctypes.c_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _i64,
         _i64, _p, _i64, _i64, ctypes.c_float, _p, _p, _p],
    ),
    "gw_source_downsample_static_pack4": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _p, _p],
    ),
    "gw_sparse_attn_fwd_dense_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int]),
    "gw_sparse_attn_fwd_dense": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64, _i64, _p, _i64p, _p, _p,
         _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, ctypes.c_int, _i64, _i64,
         ctypes.c_float, _p, _p, _sz, _p],
    ),
    "gw_sparse_attn_fwd_dense_noalloc_capacity": (_sz, []),
    "gw_sparse_attn_fwd_dense_noalloc": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64, _i64, _p, _i64p, _p, _p,
         _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p, ctypes.c_int, _i64, _i64,
         ctypes.c_float, _p, _p],
    ),
    "gw_sparse_attn_bwd_dense_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "gw_sparse_attn_bwd_dense": (
        ctypes.c_int,
        [ctypes.c_int, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64, _i64, _p, _i64p, _p, _i64p,
         _p, _p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _i64, _i64,
         ctypes.c_float, _p, _p, _sz, _p],
    ),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load the library once (raises RuntimeError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m geoweave_amd.build` "
                    "(hipcc, gfx950) before using the geoweave_amd kernels"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def exported_names() -> Sequence[str]:
    return tuple(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != GW_OK:
        msg = load().gw_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def dtype_code(dtype: torch.dtype, allow_fp32: bool = False) -> int:
    """The C ABI's dtype code. fp32 only where the entry point takes it (``allow_fp32``:
    the indexer top-k, its backward and the KL loss)."""
    if dtype == torch.bfloat16:
        return GW_DTYPE_BF16
    if dtype == torch.float16:
        return GW_DTYPE_FP16
    if allow_fp32 and dtype == torch.float32:
        return GW_DTYPE_FP32
    kinds = "bfloat16, float16 or float32" if allow_fp32 else "bfloat16 or float16"
    raise TypeError(f"unsupported dtype {dtype}; this HIP kernel takes {kinds}")


def strides3(*vals: int):
    return (ctypes.c_int64 * 3)(*[int(x) for x in vals])


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
