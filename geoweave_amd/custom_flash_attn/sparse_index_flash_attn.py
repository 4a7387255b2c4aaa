"""Sparse-index flash attention on gfx950: the drop-in for the reference module
``easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py``.

Names, argument meaning and return values follow the reference API (``:3108-3456``):

* ``sparse_index_flash_attn_func(q, k, v, kv_positions, bias=None, causal=False,
  softmax_scale=None) -> (o, attn_sum)`` with autograd (reference ``:3196-3286``);
* ``sparse_index_flash_attn_inference_func(..., return_attn=False)`` (``:3138-3163``);
* the ``[B, H, T, D]`` twins ``sparse_index_flash_attn_bhtd_func`` (``:3289-3370``) and
  ``sparse_index_flash_attn_inference_bhtd_func`` (``:3166-3193``);
* ``dense_index_flash_attn_func`` over broadcast dense positions (``:3108-3135``);
* ``sparse_index_flash_attn_value_gate_bhtd_func`` is exported as ``None``: the value-gated
  objective (reference ``:3373-3456``) is off in the presets and not built here. The
  caller imports all six names in one ``try`` block (``dsa_attention.py:29-45``) and
  checks this one for ``None`` before use (``:5202``), so it takes its own torch path.

q: ``[B, T, H, D]``, k/v: ``[B, S, H, D]`` (bthd), kv_positions: int32 ``[B, T, K]``
shared by all heads; entries outside ``[0, S)`` are masked. Preconditions are the
reference's (``:2013-2039``): fp16/bf16 inputs of one dtype, CUDA(HIP) tensors, int32
positions of shape ``(B, T, K)``, any head dim d <= 128 (the kernels are built for 64 and
128; other d run on inputs zero-padded to the next of those). ``bias`` and ``causal=True`` are rejected, as the reference's
forward kernel asserts (``:199``, ``:203``).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from .. import _lib

__all__ = [
    "sparse_index_flash_attn_func",
    "sparse_index_flash_attn_inference_func",
    "sparse_index_flash_attn_bhtd_func",
    "sparse_index_flash_attn_inference_bhtd_func",
    "dense_index_flash_attn_func",
    "sparse_index_flash_attn_value_gate_bhtd_func",
    "SparseIndexFlashAttnFunc",
    "SparseIndexFlashAttnBhtdFunc",
]


def _bthd_strides(x: torch.Tensor, layout: str):
    """(stride_b, stride_t, stride_h) of a 4-D tensor in the given logical layout."""
    if layout == "bthd":
        return x.stride(0), x.stride(1), x.stride(2)
    return x.stride(0), x.stride(2), x.stride(1)


def _dims(q, k, layout: str):
    if layout == "bthd":
        batch, seqlen_q, nheads, d = q.shape
        seqlen_k = k.shape[1]
    elif layout == "bhtd":
        batch, nheads, seqlen_q, d = q.shape
        seqlen_k = k.shape[2]
    else:
        raise ValueError(f"Unsupported q_layout: {layout}")
    return batch, seqlen_q, seqlen_k, nheads, d


def _check_inputs(q, k, v, kv_positions, bias, causal, layout):
    batch, seqlen_q, seqlen_k, nheads, d = _dims(q, k, layout)
    if layout == "bthd":
        exp_kv = (batch, seqlen_k, nheads, d)
    else:
        exp_kv = (batch, nheads, seqlen_k, d)
    if tuple(k.shape) != exp_kv or tuple(v.shape) != exp_kv:
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match {exp_kv}")
    if d > 128:
        raise ValueError("FlashAttention only support head dimensions up to 128")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("All tensors must have the same type")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("Only support fp16 and bf16")
    if not (q.is_cuda and k.is_cuda and v.is_cuda and kv_positions.is_cuda):
        raise ValueError("q, k, v and kv_positions must be GPU tensors")
    if kv_positions.dtype != torch.int32:
        raise TypeError("kv_positions must be int32")
    if kv_positions.dim() != 3 or tuple(kv_positions.shape[:2]) != (batch, seqlen_q):
        raise ValueError(
            f"kv_positions shape {tuple(kv_positions.shape)} must be (B, T, K) = ({batch}, {seqlen_q}, K)"
        )
    if bias is not None:
        raise NotImplementedError("attention bias is not supported by the sparse forward kernel")
    if causal:
        raise NotImplementedError("causal sparse-index attention is not supported")
    if d < 1:
        raise ValueError(f"head dim must be positive, got {d}")
    return batch, seqlen_q, seqlen_k, nheads, d


# Head dims the kernels are built for. Any other d <= 128 (the reference takes any d up to
# 128, sparse_index_flash_attn.py:2034) runs on q, k, v (and o, dO) zero-padded to the next
# built size: padded dims add nothing to q.k, and the outputs' padded dims are dropped.
NATIVE_HEAD_DIMS = (64, 128)


def _padded_head_dim(d: int) -> int:
    return 64 if d <= 64 else 128


def _pad_head_dim(x: torch.Tensor, dp: int) -> torch.Tensor:
    return torch.nn.functional.pad(x, (0, dp - x.shape[-1]))


# Forward: "auto" picks the masked dense pass (gw_sparse_attn_fwd_dense) when a query
# selects at least 1 / DENSE_MAX_RATIO of the keys (and, with attn_sum, K <=
# DENSE_ATTN_SUM_MAX_K), "dense" / "gather" force one path (tests and measurements). The
# dense pass costs ~ T·S, the gather ~ T·K: on MI355X they break even near S = 124·K.
# The dense kernel's 32-bit load offsets bound the K token stride and S, its grid of at most
# 65535 query blocks (whole workgroups of 8) bounds T (DENSE_MAX_*).
FORWARD_PATH = "auto"
DENSE_MAX_RATIO = 96
DENSE_ATTN_SUM_MAX_K = 1024
DENSE_MAX_K_ROW_STRIDE = 1 << 23
DENSE_MAX_S = (1 << 25) - 128
DENSE_MAX_T = 65528 * 32


def _use_dense(seqlen_k: int, num_kv: int, nheads: int, d: int, softmax_scale: float = 1.0) -> bool:
    if FORWARD_PATH == "gather" or d != 64 or not 0.0 < softmax_scale < float("inf"):
        return False
    return FORWARD_PATH == "dense" or seqlen_k <= DENSE_MAX_RATIO * num_kv


def _dense_fits(k: torch.Tensor, q_layout: str, seqlen_k: int, seqlen_q: int = 0) -> bool:
    """The dense forward's limits: K token stride and S (32-bit load offsets), T (grid)."""
    return (_bthd_strides(k, q_layout)[1] < DENSE_MAX_K_ROW_STRIDE and seqlen_k <= DENSE_MAX_S
            and seqlen_q <= DENSE_MAX_T)


def _prep(x: torch.Tensor) -> torch.Tensor:
    # Last dim contiguous and 16-byte aligned b/t/h strides (reference :3207-3209 makes
    # the last dim contiguous; the gfx950 kernel also needs 16-byte rows).
    if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:-1]) or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def _flash_attn_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    bias=None,
    causal: bool = False,
    softmax_scale: Optional[float] = None,
    return_attn: bool = True,
    q_layout: str = "bthd",
    kl_logits: Optional[torch.Tensor] = None,
    kl_eps: float = 1e-6,
    kl_row_loss: Optional[torch.Tensor] = None,
):
    """Returns (o, attn_sum | None, lse [B,T,H] fp32, softmax_scale).

    o has q's shape and dtype and is contiguous (reference :2064-2067); attn_sum is fp32
    ``[B, T, K]`` (reference :2070-2075). With ``kl_logits`` ([B, T, K], unit last stride)
    the indexer KL row losses are computed in the same launch (gw_sparse_attn_fwd_kl) into
    ``kl_row_loss`` (fp32 [B*T])."""
    batch, seqlen_q, seqlen_k, nheads, d = _check_inputs(q, k, v, kv_positions, bias, causal, q_layout)
    if d not in NATIVE_HEAD_DIMS:
        dp = _padded_head_dim(d)
        o, attn_sum, lse, scale = _flash_attn_forward(
            _pad_head_dim(q, dp), _pad_head_dim(k, dp), _pad_head_dim(v, dp), kv_positions,
            softmax_scale=softmax_scale or 1.0 / math.sqrt(d), return_attn=return_attn, q_layout=q_layout,
            kl_logits=kl_logits, kl_eps=kl_eps, kl_row_loss=kl_row_loss)
        return o[..., :d].contiguous(), attn_sum, lse, scale
    q, k, v = _prep(q), _prep(k), _prep(v)
    if kv_positions.stride(-1) != 1:
        kv_positions = kv_positions.contiguous()
    num_kv = kv_positions.shape[-1]
    softmax_scale = softmax_scale or 1.0 / math.sqrt(d)
    o = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    lse = torch.empty((batch, seqlen_q, nheads), device=q.device, dtype=torch.float32)
    attn_sum = None
    if return_attn:
        attn_sum = torch.empty((batch, seqlen_q, num_kv), device=q.device, dtype=torch.float32)
    if batch == 0 or seqlen_q == 0 or num_kv == 0:
        if attn_sum is not None:
            attn_sum.zero_()
        o.zero_()
        lse.fill_(-math.inf)
        return o, attn_sum, lse, softmax_scale
    lib = _lib.load()
    common = (
        _lib.dtype_code(q.dtype),
        q.data_ptr(), _lib.strides3(*_bthd_strides(q, q_layout)),
        k.data_ptr(), _lib.strides3(*_bthd_strides(k, q_layout)),
        v.data_ptr(), _lib.strides3(*_bthd_strides(v, q_layout)),
        kv_positions.data_ptr(), kv_positions.stride(0), kv_positions.stride(1),
        o.data_ptr(), _lib.strides3(*_bthd_strides(o, q_layout)),
        lse.data_ptr(), _lib.ptr(attn_sum),
        batch, seqlen_q, seqlen_k, nheads, d, num_kv,
        float(softmax_scale),
    )
    stream = _lib.stream_handle(q.device)
    if kl_logits is None:
        kl_args = (None, 0, 0, 0, 0.0, None)
    else:
        code = _lib.GW_DTYPE_FP32 if kl_logits.dtype == torch.float32 else _lib.dtype_code(kl_logits.dtype)
        kl_args = (kl_logits.data_ptr(), code, kl_logits.stride(0), kl_logits.stride(1), float(kl_eps),
                   kl_row_loss.data_ptr())
    if (_use_dense(seqlen_k, num_kv, nheads, d, softmax_scale) and _dense_fits(k, q_layout, seqlen_k, seqlen_q)
            and (attn_sum is None or num_kv <= DENSE_ATTN_SUM_MAX_K)):
        dense_bytes = int(lib.gw_sparse_attn_fwd_dense_workspace_size(batch, seqlen_q, seqlen_k, nheads, d, num_kv,
                                                                      int(attn_sum is not None)))
        dws = torch.empty(max(dense_bytes, 1), device=q.device, dtype=torch.uint8)
        rc = lib.gw_sparse_attn_fwd_dense(*common, *kl_args, dws.data_ptr(), dense_bytes, stream)
        _lib.check(rc, "gw_sparse_attn_fwd_dense")
        return o, attn_sum, lse, softmax_scale
    ws, ws_bytes = None, 0
    if attn_sum is not None:
        ws_bytes = int(lib.gw_sparse_attn_fwd_workspace_size(batch, seqlen_q, nheads, num_kv, 1))
        ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
    if kl_logits is None:
        rc = lib.gw_sparse_attn_fwd(*common, _lib.ptr(ws), ws_bytes, stream)
        _lib.check(rc, "gw_sparse_attn_fwd")
    else:
        rc = lib.gw_sparse_attn_fwd_kl(*common, *kl_args, _lib.ptr(ws), ws_bytes, stream)
        _lib.check(rc, "gw_sparse_attn_fwd_kl")
    return o, attn_sum, lse, softmax_scale


def _flash_attn_backward(do, q, k, v, kv_positions, o, lse, dattn_sum, softmax_scale, q_layout):
    from . import _backward

    d = q.shape[-1]
    if d not in NATIVE_HEAD_DIMS:
        dp = _padded_head_dim(d)
        if do is None:
            do = torch.zeros_like(o)
        dq, dk, dv = _backward.sparse_attn_backward(
            *(_pad_head_dim(x, dp) for x in (do, q, k, v)), kv_positions, _pad_head_dim(o, dp), lse, dattn_sum,
            softmax_scale, q_layout)
        return dq[..., :d].contiguous(), dk[..., :d].contiguous(), dv[..., :d].contiguous()
    return _backward.sparse_attn_backward(do, q, k, v, kv_positions, o, lse, dattn_sum, softmax_scale, q_layout)


class SparseIndexFlashAttnFunc(torch.autograd.Function):
    """Autograd wrapper of the bthd kernel (reference ``:3196-3283``)."""

    @staticmethod
    def forward(ctx, q, k, v, kv_positions, bias=None, causal=False, softmax_scale=None):
        # An output that takes no part in the loss (attn_sum detached before the indexer loss,
        # as the reference presets do) brings None instead of zeros: the backward then skips
        # the attn_sum term, which zeros would contribute nothing to.
        ctx.set_materialize_grads(False)
        if kv_positions.stride(-1) != 1:
            kv_positions = kv_positions.contiguous()
        o, attn_sum, lse, ctx.softmax_scale = _flash_attn_forward(
            q, k, v, kv_positions, bias=bias, causal=causal, softmax_scale=softmax_scale,
            return_attn=True, q_layout="bthd",
        )
        ctx.save_for_backward(q, k, v, kv_positions, o, lse)
        return o, attn_sum

    @staticmethod
    def backward(ctx, do, dattn_sum):
        q, k, v, kv_positions, o, lse = ctx.saved_tensors
        dq, dk, dv = _flash_attn_backward(
            do, q, k, v, kv_positions, o, lse, dattn_sum, ctx.softmax_scale, "bthd"
        )
        return dq, dk, dv, None, None, None, None


class SparseIndexFlashAttnBhtdFunc(torch.autograd.Function):
    """Autograd wrapper of the ``[B, H, T, D]`` layout (reference ``:3289-3367``)."""

    @staticmethod
    def forward(ctx, q, k, v, kv_positions, bias=None, causal=False, softmax_scale=None):
        # An output that takes no part in the loss (attn_sum detached before the indexer loss,
        # as the reference presets do) brings None instead of zeros: the backward then skips
        # the attn_sum term, which zeros would contribute nothing to.
        ctx.set_materialize_grads(False)
        if kv_positions.stride(-1) != 1:
            kv_positions = kv_positions.contiguous()
        o, attn_sum, lse, ctx.softmax_scale = _flash_attn_forward(
            q, k, v, kv_positions, bias=bias, causal=causal, softmax_scale=softmax_scale,
            return_attn=True, q_layout="bhtd",
        )
        ctx.save_for_backward(q, k, v, kv_positions, o, lse)
        return o, attn_sum

    @staticmethod
    def backward(ctx, do, dattn_sum):
        q, k, v, kv_positions, o, lse = ctx.saved_tensors
        dq, dk, dv = _flash_attn_backward(
            do, q, k, v, kv_positions, o, lse, dattn_sum, ctx.softmax_scale, "bhtd"
        )
        return dq, dk, dv, None, None, None, None


sparse_index_flash_attn_func = SparseIndexFlashAttnFunc.apply
sparse_index_flash_attn_bhtd_func = SparseIndexFlashAttnBhtdFunc.apply


@torch.inference_mode()
def sparse_index_flash_attn_inference_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    causal: bool = False,
    softmax_scale: Optional[float] = None,
    return_attn: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Inference entry that skips attn_sum unless asked (reference ``:3138-3163``)."""
    o, attn_sum, _, _ = _flash_attn_forward(
        q, k, v, kv_positions, bias=bias, causal=causal, softmax_scale=softmax_scale,
        return_attn=return_attn, q_layout="bthd",
    )
    return o, attn_sum


@torch.inference_mode()
def sparse_index_flash_attn_inference_bhtd_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_positions: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    causal: bool = False,
    softmax_scale: Optional[float] = None,
    return_attn: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """``[B, H, T, D]`` inference entry (reference ``:3166-3193``)."""
    o, attn_sum, _, _ = _flash_attn_forward(
        q, k, v, kv_positions, bias=bias, causal=causal, softmax_scale=softmax_scale,
        return_attn=return_attn, q_layout="bhtd",
    )
    return o, attn_sum


def _build_dense_kv_positions(batch: int, seqlen_q: int, seqlen_k: int, device) -> torch.Tensor:
    """Broadcast dense positions ``[B, Tq, Tk]`` with O(Tk) storage (reference ``:3108-3118``)."""
    base = torch.arange(seqlen_k, device=device, dtype=torch.int32)
    return torch.as_strided(base, size=(batch, seqlen_q, seqlen_k), stride=(0, 0, 1))


def dense_index_flash_attn_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    causal: bool = False,
    softmax_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense attention through the sparse-index kernel (reference ``:3121-3135``)."""
    batch, seqlen_q, _, _ = q.shape
    seqlen_k = k.shape[1]
    kv_positions = _build_dense_kv_positions(batch, seqlen_q, seqlen_k, q.device)
    return SparseIndexFlashAttnFunc.apply(q, k, v, kv_positions, bias, causal, softmax_scale)


# Not provided (see the module docstring): the caller falls back when it is None.
sparse_index_flash_attn_value_gate_bhtd_func = None
