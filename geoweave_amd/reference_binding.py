"""Install the gfx950 drop-ins under the reference's module names.

The reference reaches the kernels through three import sites, each in a ``try`` that
tolerates absence:

* ``easyvolcap/official_vggt/layers/indexer.py:10-14``:
  ``from easyvolcap.utils.custom_indexer import sparse_topk_indexer_func,
  sparse_topk_indexer_inference_func``;
* ``easyvolcap/official_vggt/layers/dsa_attention.py:24-27``:
  ``from easyvolcap.utils.custom_indexer.indexer_kl_fused import sparse_indexer_kl_loss``;
* ``dsa_attention.py:28-45``: the six names of
  ``easyvolcap.utils.custom_flash_attn.sparse_index_flash_attn``.

``indexer.py:8-9`` also imports ``custom_indexer.streaming_kl_autograd`` and
``custom_indexer.topk_support_autograd`` outside any ``try``; those modules (and the Triton
helpers of the real ``custom_indexer.sparse_topk_indexer`` they use) stay the reference's.
So the package ``easyvolcap.utils.custom_indexer`` is the real one: ``install()`` registers
this build's modules for the two leaf modules it replaces (before the package is imported,
so the package's own ``from .indexer_kl_fused import ...`` picks this build's loss), imports
the package, and rebinds the three exported functions on it. Call it before
``easyvolcap.official_vggt.layers.indexer`` / ``dsa_attention`` are imported: their
``from ... import`` statements bind names at import time.
"""
from __future__ import annotations

import importlib
import sys
from types import ModuleType

__all__ = ["install"]


def install(root: str = "easyvolcap.utils") -> ModuleType:
    """Returns the (real) ``{root}.custom_indexer`` package after rebinding its exports."""
    from .custom_flash_attn import sparse_index_flash_attn as attn
    from .custom_indexer import indexer_kl_fused as kl
    from .custom_indexer import sparse_topk_indexer as sti

    sys.modules[f"{root}.custom_flash_attn.sparse_index_flash_attn"] = attn
    sys.modules[f"{root}.custom_indexer.indexer_kl_fused"] = kl
    flash_pkg = importlib.import_module(f"{root}.custom_flash_attn")
    flash_pkg.sparse_index_flash_attn = attn
    pkg = importlib.import_module(f"{root}.custom_indexer")
    pkg.indexer_kl_fused = kl
    pkg.sparse_topk_indexer_func = sti.sparse_topk_indexer_func
    pkg.sparse_topk_indexer_inference_func = sti.sparse_topk_indexer_inference_func
    pkg.sparse_indexer_kl_loss = kl.sparse_indexer_kl_loss
    return pkg
