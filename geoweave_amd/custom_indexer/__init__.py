"""Lightning-indexer top-k operators (gfx950). Mirrors the export surface of the reference
package ``easyvolcap/utils/custom_indexer/__init__.py:1-13`` for the hot path:
``sparse_topk_indexer_func`` and ``sparse_topk_indexer_inference_func`` (here a real
inference entry instead of the reference's ``None``). The reference's training-loss export
``sparse_indexer_kl_loss`` is outside this path and is not provided."""
from .sparse_topk_indexer import sparse_topk_indexer_func, sparse_topk_indexer_inference_func

__all__ = ["sparse_topk_indexer_func", "sparse_topk_indexer_inference_func"]
