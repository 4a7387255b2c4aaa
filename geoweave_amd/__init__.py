"""MI355X-native (gfx950) sparse global-attention hot path of GeoWeave.

Drop-in operator modules (same names and signatures as the reference):

* ``geoweave_amd.custom_indexer``: ``sparse_topk_indexer_func`` and
  ``sparse_topk_indexer_inference_func`` (lightning-indexer score + exact top-k);
* ``geoweave_amd.custom_flash_attn.sparse_index_flash_attn``: ``sparse_index_flash_attn_func``
  and its inference / bhtd / dense variants.

All compute runs in ``libgeoweave_hip.so`` (hand-written HIP for gfx950, C ABI in
``include/geoweave_hip.h``), built with ``python -m geoweave_amd.build``.
"""

__version__ = "0.1.0"
