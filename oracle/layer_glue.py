"""fp32 CPU restatement of the DSA layer glue around the hot-path kernels: the fused
projection, per-head LayerNorm, 2D rotary embedding and the 16-bit cast.

Test infrastructure only (see ``oracle/__init__.py``).

Reference: ``DSAAttention._project_qkv_and_indexer_fused``
(``easyvolcap/official_vggt/layers/dsa_attention.py:583-625``), the q/k glue of
``DSAAttention.forward`` (``:4928-4948``), ``LightningIndexer.project``
(``easyvolcap/official_vggt/layers/indexer.py:302-328``) and
``RotaryPositionEmbedding2D`` (``easyvolcap/official_vggt/layers/rope.py:62-200``); Pi3's
``RoPE2D`` (``aidi/third_party/pi3_training/pi3/models/layers/pos_embed.py:112-160``, the
torch module the reference runs: its compiled ``cuRoPE2D`` is not part of the checkout) and
Pi3's token positions (``pi3_training.py:818-827``, ``pos_embed.py:161-173``).
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F


def rope2d_tables(max_position: int, feature_dim: int = 32, base: float = 100.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) fp32 ``[max_position, feature_dim // 2]``: ``rope.py:86-117`` (the reference
    concatenates the table with itself, ``cat(t, t)``; one copy is kept here)."""
    exponents = torch.arange(0, feature_dim, 2).float() / feature_dim
    inv_freq = 1.0 / (base ** exponents)
    positions = torch.arange(max_position, dtype=inv_freq.dtype)
    angles = torch.einsum("i,j->ij", positions, inv_freq)
    return angles.cos(), angles.sin()


def rope1d(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``rope.py:133-152``: ``x * cos[p] + cat(-x2, x1) * sin[p]`` over the last dim
    (x ``[B, H, N, d]``, positions ``[B, N]``)."""
    c = torch.cat((cos, cos), dim=-1)[positions][:, None]
    s = torch.cat((sin, sin), dim=-1)[positions][:, None]
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * c + rot * s


def rope2d(tokens: torch.Tensor, positions: torch.Tensor, base: float = 100.0) -> torch.Tensor:
    """``RotaryPositionEmbedding2D.forward`` (``rope.py:154-200``): tokens ``[B, H, N, D]``,
    positions ``[B, N, 2]`` (y, x); dims ``[0, D/2)`` rotate with y, ``[D/2, D)`` with x."""
    feature_dim = tokens.shape[-1] // 2
    cos, sin = rope2d_tables(int(positions.max()) + 1, feature_dim, base)
    vert, horiz = tokens.chunk(2, dim=-1)
    vert = rope1d(vert, positions[..., 0].long(), cos, sin)
    horiz = rope1d(horiz, positions[..., 1].long(), cos, sin)
    return torch.cat((vert, horiz), dim=-1)


def rope2d_pi3(tokens: torch.Tensor, positions: torch.Tensor, freq: float = 100.0) -> torch.Tensor:
    """Pi3's ``RoPE2D.forward`` (``pos_embed.py:112-160``) in fp32: D = dim/2 features per
    axis, ``inv_freq = 1 / freq^(arange(0, D, 2)/D)``, ``freqs = cat(t x inv_freq, t x
    inv_freq)``, the first half of the features rotated with ``positions[..., 0]`` (y) and
    the second with ``positions[..., 1]`` (x), each by ``x cos + rotate_half(x) sin`` with
    ``rotate_half(x) = cat(-x2, x1)``. tokens ``[B, H, N, dim]``, positions ``[B, N, 2]``."""
    D = tokens.shape[-1] // 2
    n_pos = int(positions.max()) + 1
    inv_freq = 1.0 / (freq ** (torch.arange(0, D, 2).float() / D))
    t = torch.arange(n_pos, dtype=inv_freq.dtype)
    freqs = torch.einsum("i,j->ij", t, inv_freq)
    freqs = torch.cat((freqs, freqs), dim=-1)
    cos, sin = freqs.cos(), freqs.sin()

    def rotate_half(x):
        return torch.cat((-x[..., x.shape[-1] // 2:], x[..., :x.shape[-1] // 2]), dim=-1)

    def apply_1d(x, p):
        c = F.embedding(p, cos)[:, None, :, :]
        s_ = F.embedding(p, sin)[:, None, :, :]
        return x * c + rotate_half(x) * s_

    y, x = tokens.float().chunk(2, dim=-1)
    return torch.cat((apply_1d(y, positions[:, :, 0].long()), apply_1d(x, positions[:, :, 1].long())), dim=-1)


def pi3_positions(batch_views: int, grid_h: int, grid_w: int, n_special: int = 5) -> torch.Tensor:
    """int64 ``[batch_views, n_special + grid_h * grid_w, 2]``: Pi3's decoder positions
    (``pi3_training.py:818-827``): the (y, x) patch grid of ``PositionGetter``
    (``pos_embed.py:161-173``, row-major ``cartesian_prod(y, x)``) plus one, after
    ``n_special`` register tokens at (0, 0)."""
    ys = torch.arange(grid_h).repeat_interleave(grid_w)
    xs = torch.arange(grid_w).repeat(grid_h)
    grid = torch.stack([ys, xs], dim=-1) + 1
    special = torch.zeros(n_special, 2, dtype=grid.dtype)
    return torch.cat([special, grid], dim=0).expand(batch_views, -1, -1).clone()


def fused_projection_glue(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    dims: Dict[str, int],
    norms: Dict[str, Optional[Tuple[torch.Tensor, torch.Tensor]]],
    pos: Optional[torch.Tensor],
    ln_eps: float = 1e-5,
    rope_base: float = 100.0,
    y: Optional[torch.Tensor] = None,
    rope=None,
):
    """(q, k, v, idx_q, idx_k, idx_w) in fp32, q/k/v ``[B, N, H, D]``, idx_q/idx_k
    ``[B, N, Hi, Di]``, idx_w ``[B, N, Hi]``.

    ``y = x W^T + b`` with W the concatenation ``[qkv | idx_q | idx_k | idx_w]``
    (``dsa_attention.py:590-600``; pass ``y`` to start from a given projection). q/k:
    ``q_norm``/``k_norm`` LayerNorm over the head dim, then rope (``:4935-4940``); indexer
    k: ``k_norm`` then rope, indexer q: rope (``:606-618``). ``norms`` maps 'q', 'k',
    'idx_k' to (weight, bias) or None (identity). ``rope``: the rotation ``(tokens [B, H, N,
    D], pos, base) -> tokens`` (default ``rope2d``, VGGT's; ``rope2d_pi3`` for Pi3's).
    """
    H, D, Hi, Di = dims["H"], dims["D"], dims["Hi"], dims["Di"]
    if y is None:
        y = F.linear(x.float(), weight.float(), None if bias is None else bias.float())
    y = y.float()
    B, N = y.shape[0], y.shape[1]
    c = 0
    q = y[..., c:c + H * D].reshape(B, N, H, D); c += H * D
    k = y[..., c:c + H * D].reshape(B, N, H, D); c += H * D
    v = y[..., c:c + H * D].reshape(B, N, H, D); c += H * D
    iq = y[..., c:c + Hi * Di].reshape(B, N, Hi, Di); c += Hi * Di
    ik = y[..., c:c + Hi * Di].reshape(B, N, Hi, Di); c += Hi * Di
    iw = y[..., c:c + Hi].reshape(B, N, Hi)

    def ln(t, key):
        p = norms.get(key)
        if p is None:
            return t
        return F.layer_norm(t, (t.shape[-1],), p[0].float(), p[1].float(), ln_eps)

    q, k, ik = ln(q, "q"), ln(k, "k"), ln(ik, "idx_k")
    if pos is not None:
        rot = rope2d if rope is None else rope
        rp = lambda t: rot(t.permute(0, 2, 1, 3), pos, rope_base).permute(0, 2, 1, 3)
        q, k, iq, ik = rp(q), rp(k), rp(iq), rp(ik)
    return q, k, v, iq, ik, iw
