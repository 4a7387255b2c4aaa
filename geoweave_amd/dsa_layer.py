"""The sparse global-attention layer on gfx950: fused projection, layer glue, indexer
top-k and sparse attention.

Counterpart of the sparse inference path of the reference ``DSAAttention``
(``easyvolcap/official_vggt/layers/dsa_attention.py:47-5403``) with its
``LightningIndexer`` (``easyvolcap/official_vggt/layers/indexer.py:40-330``), keeping the
reference's parameter names (``qkv``, ``q_norm``, ``k_norm``, ``proj``,
``indexer.{q_proj, k_proj, w_proj, k_norm}``) so that its state dict loads as is:

1. ``y = x W^T + b`` with ``W = [qkv | indexer q | indexer k | indexer w]``: one library
   GEMM (``_project_qkv_and_indexer_fused``, ``dsa_attention.py:583-625``); the fused
   weight's row count is padded to a multiple of 8 so every column block starts on a
   16-byte boundary.
2. ``gw_dsa_glue_fwd``: per-head LayerNorm, 2D RoPE and the 16-bit cast of q/k (attention)
   and q/k/w (indexer) in one pass (``:4928-4948``, ``indexer.py:302-328``); v is read in
   place from ``y`` through strides.
3. ``gw_indexer_topk_fwd`` (top-k), ``gw_sparse_attn_fwd`` (attention), then ``proj``.

The layer runs in the activations' 16-bit dtype (bf16 by default); the glue's LayerNorm
and RoPE are fp32 math on the 16-bit projection with one rounding at the end. With
``score_dtype`` set (the reference preset's ``"score_dtype": "float16"`` under bf16
activations, ``geoweave/configs/vggt.json:35``), the attention q/k/v and the indexer q/k/w
are cast to it after the glue and the indexer and attention run in it; their output is cast
back to the activations' dtype before ``proj`` (``dsa_attention.py:4943-4948,5473``,
``:617-620``).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .custom_flash_attn.sparse_index_flash_attn import (
    sparse_index_flash_attn_func,
    sparse_index_flash_attn_inference_func,
)
from .custom_indexer.sparse_topk_indexer import sparse_topk_indexer_func, sparse_topk_indexer_inference_func
from . import source_downsample as sdown

__all__ = ["GlueLayout", "rope2d_tables", "dsa_glue_forward", "sparse_attention_streaming",
           "LightningIndexerProjections", "SparseGlobalAttention", "parse_score_dtype", "rope_base_from_pos_type",
           "pi3_global_attention", "grid_positions"]


def rope_base_from_pos_type(pos_type: str) -> Optional[float]:
    """Pi3's ``pos_type`` (``pi3_training.py:163-167``): "rope<freq>" (e.g. "rope100") gives
    the rotary base ``freq``; any other type has no rotary embedding (None)."""
    if isinstance(pos_type, str) and pos_type.startswith("rope"):
        return float(pos_type[len("rope"):])
    return None


def grid_positions(batch_views: int, grid_h: int, grid_w: int, n_special: int = 5, device=None) -> torch.Tensor:
    """int32 ``[batch_views, n_special + grid_h * grid_w, 2]`` token positions shared by VGGT
    and Pi3 (``aggregator.py:521-526``; Pi3 ``pi3_training.py:818-827``): ``n_special``
    camera/register tokens at (0, 0), then the (y, x) patch grid plus one, row-major. For a
    global-attention layer over S views, reshape to ``[B, S * tokens, 2]``."""
    ys = torch.arange(grid_h, device=device).repeat_interleave(grid_w)
    xs = torch.arange(grid_w, device=device).repeat(grid_h)
    grid = torch.stack([ys, xs], dim=-1) + 1
    special = torch.zeros(n_special, 2, dtype=grid.dtype, device=device)
    return torch.cat([special, grid], 0).to(torch.int32).expand(batch_views, -1, -1).contiguous()


def parse_score_dtype(value) -> Optional[torch.dtype]:
    """The reference's dtype spelling (``DSAAttention._parse_dtype``,
    ``dsa_attention.py:503-518``): a torch dtype, or "fp16"/"float16"/"half"/"f16",
    "bf16"/"bfloat16", "fp32"/"float32"/"f32"; None, "", "none" and (as in the reference)
    any other string mean "the activations' dtype". With float32 the indexer computes in
    fp32 and the attention casts its fp32 q/k/v to bfloat16, as the reference does
    (``dsa_attention.py:4943-4948,5296-5300``)."""
    if value is None:
        return None
    if isinstance(value, str):
        text = value.strip().lower()
        if text in ("", "none"):
            return None
        table = {"fp16": torch.float16, "float16": torch.float16, "half": torch.float16, "f16": torch.float16,
                 "bf16": torch.bfloat16, "bfloat16": torch.bfloat16,
                 "fp32": torch.float32, "float32": torch.float32, "f32": torch.float32}
        if text not in table:
            return None
        value = table[text]
    if not isinstance(value, torch.dtype):
        raise TypeError(f"score_dtype must be a torch dtype or a string, not {type(value).__name__}")
    if value not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"score_dtype {value} is not supported: the indexer takes bfloat16, float16 or "
                        "float32 and the attention bfloat16 or float16")
    return value


class GlueLayout:
    """Column blocks of the fused projection output (reference ``dsa_attention.py:590-600``);
    ``Hi = 0`` is a dense attention layer's plain qkv projection."""

    def __init__(self, H: int, D: int, Hi: int, Di: int):
        if D != 64 or Di != 64:
            raise NotImplementedError("the glue kernel handles 64-wide heads")
        self.H, self.D, self.Hi, self.Di = H, D, Hi, Di
        self.q_off = 0
        self.k_off = H * D
        self.v_off = 2 * H * D
        self.iq_off = 3 * H * D
        self.ik_off = self.iq_off + Hi * Di
        self.iw_off = self.ik_off + Hi * Di
        self.width = self.iw_off + Hi
        self.ldy = (self.width + 7) // 8 * 8


_ROPE_CACHE = {}


def rope2d_tables(max_position: int, base: float, device, feature_dim: int = 32) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 (cos, sin) ``[max_position, feature_dim // 2]``, built as
    ``RotaryPositionEmbedding2D._compute_frequency_components`` builds them (``rope.py:86-117``)
    for fp32 tokens (one copy of the reference's ``cat(t, t)``), and cached per
    (length, base, device) as the reference caches them (``rope.py:101-115``)."""
    key = (int(max_position), float(base), str(torch.device(device)), int(feature_dim))
    hit = _ROPE_CACHE.get(key)
    if hit is None:
        hit = _rope2d_tables(max_position, base, device, feature_dim)
        _ROPE_CACHE[key] = hit
    return hit


def _rope2d_tables(max_position: int, base: float, device, feature_dim: int):
    exponents = torch.arange(0, feature_dim, 2, device=device).float() / feature_dim
    inv_freq = 1.0 / (base ** exponents)
    positions = torch.arange(max_position, device=device, dtype=inv_freq.dtype)
    angles = torch.einsum("i,j->ij", positions, inv_freq)
    return angles.cos().contiguous(), angles.sin().contiguous()


def _ln_params(norm: Optional[nn.Module]):
    if norm is None or isinstance(norm, nn.Identity):
        return None, None
    if not isinstance(norm, nn.LayerNorm) or norm.normalized_shape != (64,):
        raise NotImplementedError("q/k norms must be LayerNorm(64) or Identity")
    w = norm.weight.detach().float().contiguous() if norm.weight is not None else None
    b = norm.bias.detach().float().contiguous() if norm.bias is not None else None
    if w is None or b is None:
        dev = norm.weight.device if norm.weight is not None else None
        w = torch.ones(64, device=dev) if w is None else w
        b = torch.zeros(64, device=w.device) if b is None else b
    return w, b


def dsa_glue_forward(
    y: torch.Tensor,
    layout: GlueLayout,
    q_norm=(None, None),
    k_norm=(None, None),
    idx_k_norm=(None, None),
    ln_eps: float = 1e-5,
    pos: Optional[torch.Tensor] = None,
    rope_base: float = 100.0,
    rope_len: Optional[int] = None,
):
    """(q, k, v, idx_q, idx_k, idx_w) from the fused projection ``y [B, N, ldy]`` via
    ``gw_dsa_glue_fwd``. q/k ``[B, N, H, 64]`` and idx_q/idx_k ``[B, N, Hi, 64]`` are new
    contiguous tensors, idx_w ``[B, N, Hi]``; v is a strided view of ``y``. ``pos`` is
    ``[B, N, 2]`` (y, x) integer positions or None (no rope); ``rope_len`` is the table
    length (default ``max(pos) + 1`` like the reference, ``rope.py:190``, which reads it on
    the host)."""
    if y.dim() != 3 or y.shape[-1] != layout.ldy or y.stride(-1) != 1 or y.stride(1) != layout.ldy:
        raise ValueError(f"y must be a contiguous [B, N, {layout.ldy}] projection")
    if not y.is_cuda:
        raise ValueError("y must be a GPU tensor")
    B, N = y.shape[0], y.shape[1]
    H, Hi = layout.H, layout.Hi
    dev = y.device
    q = torch.empty(B, N, H, 64, device=dev, dtype=y.dtype)
    k = torch.empty_like(q)
    iq = torch.empty(B, N, Hi, 64, device=dev, dtype=y.dtype) if Hi else None
    ik = torch.empty_like(iq) if Hi else None
    iw = torch.empty(B, N, Hi, device=dev, dtype=y.dtype) if Hi else None
    pos32 = cos = sin = None
    n_rope = 0
    if pos is not None:
        if tuple(pos.shape) != (B, N, 2):
            raise ValueError(f"pos shape {tuple(pos.shape)} != ({B}, {N}, 2)")
        pos32 = pos.to(device=dev, dtype=torch.int32).contiguous()
        n_rope = int(rope_len) if rope_len is not None else int(pos32.max()) + 1
        cos, sin = rope2d_tables(n_rope, rope_base, dev)
    lib = _lib.load()
    _lib.check(
        lib.gw_dsa_glue_fwd(
            _lib.dtype_code(y.dtype), y.data_ptr(), B * N, layout.ldy, layout.q_off, layout.k_off,
            layout.iq_off, layout.ik_off, layout.iw_off, H, Hi, 64,
            _lib.ptr(q_norm[0]), _lib.ptr(q_norm[1]), _lib.ptr(k_norm[0]), _lib.ptr(k_norm[1]),
            _lib.ptr(idx_k_norm[0]), _lib.ptr(idx_k_norm[1]), float(ln_eps),
            _lib.ptr(pos32), _lib.ptr(cos), _lib.ptr(sin), n_rope,
            q.data_ptr(), k.data_ptr(), _lib.ptr(iq), _lib.ptr(ik), _lib.ptr(iw),
            _lib.stream_handle(dev),
        ),
        "gw_dsa_glue_fwd",
    )
    v = y[..., layout.v_off:layout.v_off + H * 64].view(B, N, H, 64)
    return q, k, v, iq, ik, iw


def sparse_attention_streaming(q, k, v, idx_q, idx_k, idx_w, topk: int, query_chunk: int,
                               indexer_scale: float, softmax_scale: float,
                               source_downsample: Optional["sdown.SourceDownsample"] = None) -> torch.Tensor:
    """Indexer top-k and sparse attention ``query_chunk`` queries at a time (reference
    ``DSAAttention._run_sparse_streaming_direct``, ``dsa_attention.py:1017-1283``): each
    chunk's top-k indices live only while its attention runs, so peak memory for indices and
    the indexer workspace scales with the chunk, not with N. q/idx_q ``[B, N, ...]``,
    k/v/idx_k/idx_w over all keys. Returns o ``[B, N, H, D]``.

    ``source_downsample``: select each chunk's keys with the coarse selector (pooled keys built
    once for all chunks, as the reference's stream does, ``dsa_attention.py:1369-1435``). With
    qk_sym_x2_broadcast the outer chunk is the selector's own query chunk
    (``min(N, source_downsample_query_chunk)``, falling back to ``query_chunk`` when that is 0;
    ``dsa_attention.py:870-881,1127-1136``), because its coarse queries pool the tokens of a
    chunk's source cells.

    Rows are independent for the full indexer and for the legacy and subcell_static_pack4
    selectors, so those give the unchunked path's rows. exact_rerank and subcell_top1 (retries
    per selector chunk, counted from the outer chunk's start) and qk_sym_x2_broadcast (query
    cells per chunk) depend on the chunking, as in the reference's stream."""
    B, N = q.shape[0], q.shape[1]
    out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    empty = idx_q.new_empty(0)
    prepared = None
    if source_downsample is not None and int(source_downsample.factor) > 1:
        prepared = sdown.prepare(idx_k, idx_w, source_downsample)
        if prepared is not None and prepared.strategy == "qk_sym_x2_broadcast":
            qc = int(source_downsample.query_chunk or 0)
            query_chunk = min(N, qc if qc > 0 else int(query_chunk))
    for s0 in range(0, N, query_chunk):
        s1 = min(s0 + query_chunk, N)
        idx = None
        if prepared is not None:
            idx = sdown.select_topk(idx_q[:, s0:s1], idx_k, idx_w, topk, indexer_scale, source_downsample,
                                    prepared=prepared, q_offset=s0)
        if idx is None:
            idx, _ = sparse_topk_indexer_inference_func(idx_q[:, s0:s1], idx_k, idx_w, empty, topk, indexer_scale,
                                                        256, 0)
        o, _ = sparse_index_flash_attn_inference_func(q[:, s0:s1], k, v, idx, softmax_scale=softmax_scale)
        out[:, s0:s1] = o
    return out


def _glue_args(y, layout, norms, ln_eps, pos32, cos, sin, n_rope):
    B, N = y.shape[0], y.shape[1]
    (qw, qb), (kw, kb), (iw_, ib) = norms
    return [_lib.dtype_code(y.dtype), y.data_ptr(), B * N, layout.ldy, layout.q_off, layout.k_off,
            layout.iq_off, layout.ik_off, layout.iw_off, layout.H, layout.Hi, 64,
            _lib.ptr(qw), _lib.ptr(qb), _lib.ptr(kw), _lib.ptr(kb), _lib.ptr(iw_), _lib.ptr(ib), float(ln_eps),
            _lib.ptr(pos32), _lib.ptr(cos), _lib.ptr(sin), n_rope]


class GlueFunction(torch.autograd.Function):
    """Autograd wrapper of the glue: ``forward(y, qn_w, qn_b, kn_w, kn_b, ikn_w, ikn_b,
    layout, ln_eps, pos32, cos, sin, n_rope) -> (q, k, idx_q, idx_k, idx_w)``; the backward
    (``gw_dsa_glue_bwd``) returns dy (zero in the v block and the padding, where the v
    view's own gradient is added by autograd) and the LayerNorm weight/bias gradients. The
    LayerNorm parameters are fp32 tensors (pass ``param.float()`` to train them)."""

    @staticmethod
    def forward(ctx, y, qn_w, qn_b, kn_w, kn_b, ikn_w, ikn_b, layout, ln_eps, pos32, cos, sin, n_rope):
        B, N = y.shape[0], y.shape[1]
        H, Hi = layout.H, layout.Hi
        q = torch.empty(B, N, H, 64, device=y.device, dtype=y.dtype)
        k = torch.empty_like(q)
        iq = torch.empty(B, N, Hi, 64, device=y.device, dtype=y.dtype)
        ik = torch.empty_like(iq)
        iw = torch.empty(B, N, Hi, device=y.device, dtype=y.dtype)
        norms = ((qn_w, qn_b), (kn_w, kn_b), (ikn_w, ikn_b))
        lib = _lib.load()
        _lib.check(lib.gw_dsa_glue_fwd(*_glue_args(y, layout, norms, ln_eps, pos32, cos, sin, n_rope),
                                       q.data_ptr(), k.data_ptr(), iq.data_ptr(), ik.data_ptr(), iw.data_ptr(),
                                       _lib.stream_handle(y.device)), "gw_dsa_glue_fwd")
        ctx.save_for_backward(y, qn_w, qn_b, kn_w, kn_b, ikn_w, ikn_b, pos32, cos, sin)
        ctx.layout, ctx.ln_eps, ctx.n_rope = layout, ln_eps, n_rope
        ctx.has_norm = (qn_w is not None, kn_w is not None, ikn_w is not None)
        return q, k, iq, ik, iw

    @staticmethod
    def backward(ctx, dq, dk, diq, dik, diw):
        y, qn_w, qn_b, kn_w, kn_b, ikn_w, ikn_b, pos32, cos, sin = ctx.saved_tensors
        layout = ctx.layout
        B, N = y.shape[0], y.shape[1]
        grads = []
        for g, shape in ((dq, (B, N, layout.H, 64)), (dk, (B, N, layout.H, 64)), (diq, (B, N, layout.Hi, 64)),
                         (dik, (B, N, layout.Hi, 64)), (diw, (B, N, layout.Hi))):
            g = torch.zeros(shape, device=y.device, dtype=y.dtype) if g is None else g.to(y.dtype).contiguous()
            grads.append(g)
        dy = torch.zeros_like(y)
        dln = torch.empty(3, 2, 64, device=y.device, dtype=torch.float32)
        lib = _lib.load()
        nbytes = lib.gw_dsa_glue_bwd_workspace_size(B * N, layout.H, layout.Hi)
        ws = torch.empty(nbytes, device=y.device, dtype=torch.uint8)
        norms = ((qn_w, qn_b), (kn_w, kn_b), (ikn_w, ikn_b))
        _lib.check(lib.gw_dsa_glue_bwd(*_glue_args(y, layout, norms, ctx.ln_eps, pos32, cos, sin, ctx.n_rope),
                                       *[g.data_ptr() for g in grads], dy.data_ptr(), dln.data_ptr(), ws.data_ptr(),
                                       nbytes, _lib.stream_handle(y.device)), "gw_dsa_glue_bwd")
        out = [dy]
        for t, has in enumerate(ctx.has_norm):
            out += [dln[t, 0], dln[t, 1]] if has else [None, None]
        return (*out, None, None, None, None, None, None)


class LightningIndexerProjections(nn.Module):
    """Parameters of the reference ``LightningIndexer`` (``indexer.py:55-61``): q/k/w
    projections and the k LayerNorm; the gate starts at w = 1 (``:63-68``)."""

    def __init__(self, dim: int, n_heads: int = 4, head_dim: int = 64, qk_norm: bool = True):
        super().__init__()
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.q_proj = nn.Linear(dim, n_heads * head_dim)
        self.k_proj = nn.Linear(dim, n_heads * head_dim)
        self.w_proj = nn.Linear(dim, n_heads)
        nn.init.zeros_(self.w_proj.weight)
        nn.init.ones_(self.w_proj.bias)
        self.k_norm = nn.LayerNorm(head_dim) if qk_norm else nn.Identity()
        self.scale = head_dim ** -0.5


class SparseGlobalAttention(nn.Module):
    """Sparse global attention (inference): ``forward(x [B, N, dim], pos [B, N, 2] | None)
    -> [B, N, dim]``. Each query attends to the ``topk`` keys its lightning indexer ranks
    highest (``min(topk, N)``, reference ``dsa_attention.py:4996``)."""

    def __init__(self, dim: int = 1024, num_heads: int = 16, qkv_bias: bool = True, proj_bias: bool = True,
                 qk_norm: bool = True, rope_base: Optional[float] = 100.0, indexer_heads: int = 4,
                 indexer_dim: int = 64, topk: int = 1024, score_dtype=None):
        super().__init__()
        self.dim = dim
        self.score_dtype = parse_score_dtype(score_dtype)
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.qkv = nn.Linear(dim, 3 * dim, bias=qkv_bias)
        self.q_norm = nn.LayerNorm(self.head_dim) if qk_norm else nn.Identity()
        self.k_norm = nn.LayerNorm(self.head_dim) if qk_norm else nn.Identity()
        self.proj = nn.Linear(dim, dim, bias=proj_bias)
        self.indexer = LightningIndexerProjections(dim, indexer_heads, indexer_dim, qk_norm)
        self.rope_base = rope_base
        self.topk = topk
        self.layout = GlueLayout(num_heads, self.head_dim, indexer_heads, indexer_dim)
        self._fused = None

    def _to_score_dtype(self, x_dtype: torch.dtype, q, k, v, iq, ik, iw):
        """Attention q/k/v and indexer q/k/w in the score dtype (``dsa_attention.py:4943-4948``,
        ``indexer.py:321-326``); a float32 score dtype reaches the attention as bfloat16
        (``dsa_attention.py:5296-5300``: fp32 q/k/v become bf16 before the sparse kernel)."""
        sd = self.score_dtype
        if sd is None or sd == x_dtype:
            return q, k, v, iq, ik, iw
        ad = torch.bfloat16 if sd == torch.float32 else sd
        cast = lambda t, dt: None if t is None else t.to(dt)  # noqa: E731
        return cast(q, ad), cast(k, ad), cast(v, ad), cast(iq, sd), cast(ik, sd), cast(iw, sd)

    def fused_projection(self, dtype: torch.dtype):
        """(W [ldy, dim], b [ldy]) in ``dtype``: ``[qkv | q_proj | k_proj | w_proj]`` plus zero
        rows up to ``ldy`` (``_get_fused_proj_params``, ``dsa_attention.py:583-600``). Cached
        until a parameter changes."""
        lins = (self.qkv, self.indexer.q_proj, self.indexer.k_proj, self.indexer.w_proj)
        key = (dtype,) + tuple((l.weight.data_ptr(), l.weight._version,
                                0 if l.bias is None else l.bias._version) for l in lins)
        if self._fused is not None and self._fused[0] == key:
            return self._fused[1], self._fused[2]
        pad = self.layout.ldy - self.layout.width
        w = torch.cat([l.weight.detach() for l in lins], 0)
        b = torch.cat([l.bias.detach() if l.bias is not None else torch.zeros(l.out_features, device=w.device)
                       for l in lins], 0)
        if pad:
            w = torch.cat([w, w.new_zeros(pad, w.shape[1])], 0)
            b = torch.cat([b, b.new_zeros(pad)], 0)
        w, b = w.to(dtype).contiguous(), b.to(dtype).contiguous()
        self._fused = (key, w, b)
        return w, b

    @torch.no_grad()
    def forward(self, x: torch.Tensor, pos: Optional[torch.Tensor] = None, topk: Optional[int] = None,
                return_topk: bool = False, topk_indices: Optional[torch.Tensor] = None,
                rope_len: Optional[int] = None, query_chunk: Optional[int] = None,
                source_downsample: Optional["sdown.SourceDownsample"] = None):
        """``topk_indices`` (int32 ``[B, N, >= k]``): use another layer's selection and skip
        this layer's indexer (the reference's ``reuse_topk_indices``,
        ``dsa_attention.py:5014-5032``). ``rope_len``: rotary table length (default
        ``max(pos) + 1``, read on the host; pass it to keep the forward free of host syncs,
        e.g. under graph capture). ``query_chunk``: select and attend ``query_chunk`` queries
        at a time (the reference's query-chunked sparse stream, ``dsa_attention.py:1017-1283``):
        the same result with the indexer workspace and the index tensor bounded by the chunk;
        ``return_topk`` then returns None for the indices. ``source_downsample``
        (``source_downsample.SourceDownsample``): select keys with the approximate coarse
        selector over pooled keys (the reference's ``source_downsample_*`` indexer options,
        inference only, ``dsa_attention.py:4279-4318``); the full indexer runs when its
        layout does not describe this input."""
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise TypeError("SparseGlobalAttention runs in bfloat16 or float16")
        B, N, _ = x.shape
        w, b = self.fused_projection(x.dtype)
        y = F.linear(x, w, b)
        q, k, v, iq, ik, iw = dsa_glue_forward(
            y, self.layout, _ln_params(self.q_norm), _ln_params(self.k_norm), _ln_params(self.indexer.k_norm),
            self.q_norm.eps if isinstance(self.q_norm, nn.LayerNorm) else 1e-5,
            pos if self.rope_base else None, self.rope_base or 100.0, rope_len)
        q, k, v, iq, ik, iw = self._to_score_dtype(x.dtype, q, k, v, iq, ik, iw)
        kk = min(int(topk or self.topk), N)
        if query_chunk is not None and 0 < int(query_chunk) < N and topk_indices is None:
            o = sparse_attention_streaming(q, k, v, iq, ik, iw, kk, int(query_chunk), float(self.indexer.scale),
                                           self.scale, source_downsample).to(x.dtype)
            out = F.linear(o.reshape(B, N, self.dim), self.proj.weight.to(x.dtype),
                           None if self.proj.bias is None else self.proj.bias.to(x.dtype))
            return (out, None) if return_topk else out
        if topk_indices is not None:
            if topk_indices.dim() != 3 or tuple(topk_indices.shape[:2]) != (B, N) or topk_indices.shape[2] < kk:
                raise ValueError(f"reused top-k indices {tuple(topk_indices.shape)} do not cover ({B}, {N}, {kk})")
            idx = topk_indices[..., :kk]
            if idx.dtype != torch.int32:
                idx = idx.to(torch.int32)
        else:
            idx = None
            if source_downsample is not None:
                idx = sdown.select_topk(iq, ik, iw, kk, float(self.indexer.scale), source_downsample)
            if idx is None:
                idx, _ = sparse_topk_indexer_inference_func(iq, ik, iw, iq.new_empty(0), kk,
                                                            float(self.indexer.scale), 256, 0)
        o, _ = sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=self.scale)
        o = o.to(x.dtype)
        out = F.linear(o.reshape(B, N, self.dim), self.proj.weight.to(x.dtype),
                       None if self.proj.bias is None else self.proj.bias.to(x.dtype))
        return (out, idx) if return_topk else out

    def forward_train(self, x: torch.Tensor, pos: Optional[torch.Tensor] = None, topk: Optional[int] = None,
                      rope_len: Optional[int] = None):
        """Differentiable forward (training): ``-> (out, attn_sum, topk_scores, topk_indices)``.
        Gradients reach x and every parameter: the fused projection (autograd of the GEMM),
        the glue (``GlueFunction``: ``gw_dsa_glue_bwd``), the attention
        (``sparse_index_flash_attn_func``) and, through ``topk_scores``, the indexer
        (``sparse_topk_indexer_func``); ``attn_sum`` and ``topk_scores`` feed the indexer KL
        loss as in ``dsa_attention.py:5404-5411``."""
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise TypeError("SparseGlobalAttention runs in bfloat16 or float16")
        B, N, _ = x.shape
        lins = (self.qkv, self.indexer.q_proj, self.indexer.k_proj, self.indexer.w_proj)
        pad = self.layout.ldy - self.layout.width
        w = torch.cat([l.weight for l in lins] + ([x.new_zeros(pad, self.dim)] if pad else []), 0).to(x.dtype)
        b = torch.cat([l.bias for l in lins] + ([x.new_zeros(pad)] if pad else []), 0).to(x.dtype)
        y = F.linear(x, w, b)
        lay = self.layout
        pos32 = cos = sin = None
        n_rope = 0
        if pos is not None and self.rope_base:
            pos32 = pos.to(device=x.device, dtype=torch.int32).contiguous()
            n_rope = int(rope_len) if rope_len is not None else int(pos32.max()) + 1
            cos, sin = rope2d_tables(n_rope, self.rope_base, x.device)

        def ln(norm):
            if isinstance(norm, nn.Identity):
                return None, None
            return norm.weight.float(), norm.bias.float()

        eps = self.q_norm.eps if isinstance(self.q_norm, nn.LayerNorm) else 1e-5
        q, k, iq, ik, iw = GlueFunction.apply(y, *ln(self.q_norm), *ln(self.k_norm), *ln(self.indexer.k_norm), lay, eps,
                                              pos32, cos, sin, n_rope)
        v = y[..., lay.v_off:lay.v_off + lay.H * 64].view(B, N, lay.H, 64)
        q, k, v, iq, ik, iw = self._to_score_dtype(x.dtype, q, k, v, iq, ik, iw)
        kk = min(int(topk or self.topk), N)
        idx, scores = sparse_topk_indexer_func(iq, ik, iw, iq.new_empty(0), kk, float(self.indexer.scale), 256, 0)
        o, attn = sparse_index_flash_attn_func(q, k, v, idx, None, False, self.scale)
        o = o.to(x.dtype)
        out = F.linear(o.reshape(B, N, self.dim), self.proj.weight.to(x.dtype),
                       None if self.proj.bias is None else self.proj.bias.to(x.dtype))
        return out, attn, scores, idx


def pi3_global_attention(dim: int = 1024, num_heads: int = 16, pos_type: str = "rope100", topk: int = 1024,
                         indexer_heads: int = 4, indexer_dim: int = 64, score_dtype="float16") -> SparseGlobalAttention:
    """The sparse global attention of Pi3's DSA decoder blocks (``DSABlockRope``,
    ``aidi/third_party/pi3_training/pi3/models/layers/block.py:345-447``, built by
    ``pi3_training.py:245-275`` for the layers of ``indexer_layers``, 9-17 in
    ``geoweave/configs/pi3.json``): qkv bias on, per-head q/k LayerNorm, Pi3's ``RoPE2D`` with
    the base of ``pos_type`` (the same rotation as VGGT's: frequencies base^(-2i/32) per
    32-dim half, y then x), indexer 4 x 64 with top-k 1024, and the preset's fp16 scores."""
    return SparseGlobalAttention(dim, num_heads, qkv_bias=True, proj_bias=True, qk_norm=True,
                                 rope_base=rope_base_from_pos_type(pos_type), indexer_heads=indexer_heads,
                                 indexer_dim=indexer_dim, topk=topk, score_dtype=score_dtype)
