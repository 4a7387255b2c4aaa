"""Lightning-indexer operators (gfx950). Mirrors the export surface of the reference
package ``easyvolcap/utils/custom_indexer/__init__.py:1-13``: ``sparse_topk_indexer_func``,
``sparse_topk_indexer_inference_func`` (here a real inference entry instead of the
reference's ``None``) and the training loss ``sparse_indexer_kl_loss``."""
from .indexer_kl_fused import sparse_indexer_kl_loss
from .sparse_topk_indexer import sparse_topk_indexer_func, sparse_topk_indexer_inference_func

__all__ = ["sparse_topk_indexer_func", "sparse_topk_indexer_inference_func", "sparse_indexer_kl_loss"]
