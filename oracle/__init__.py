"""CPU oracle for GeoWeave's sparse global-attention hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``geoweave_amd``) imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or, in the bench, as the timed CPU
baseline), never as the thing measured on the GPU.

The oracle restates, in plain fp32 PyTorch on the CPU, the reference's own ``--backend
torch`` path (reference: ``geoweave/inference.py:56-58`` sets ``use_topk_kernel=False``,
``use_sparse_flash_attn=False``, ``score_dtype='float32'``):

* ``indexer.indexer_scores`` / ``indexer.indexer_topk``: ``LightningIndexer._compute_scores``
  + ``scores.topk(k, sorted=False)`` (reference
  ``easyvolcap/official_vggt/layers/indexer.py:383-466,600-603``);
* ``indexer.indexer_topk_bwd``: gradient of the selected scores w.r.t. q, k, w
  (reference ``easyvolcap/utils/custom_indexer/sparse_topk_indexer.py:1847-1944``);
* ``attention.sparse_attention``: gathered sparse softmax attention with invalid-position
  masking and ``attn_sum`` (reference ``tests/sparse_index_flash_attn_tests.py:47-71``,
  ``easyvolcap/official_vggt/layers/dsa_attention.py:4717-4753,1774-1816``);
* ``kl_loss.kl_row_losses`` / ``kl_loss.kl_loss_bwd``: the indexer KL training loss and its
  explicit gradient (reference ``easyvolcap/utils/custom_indexer/indexer_kl_fused.py:8-298``),
  pinned by scipy.stats.entropy (eps = 0), autograd and finite differences;
* ``source_downsample``: the source-downsample coarse selector (layout, pooled keys,
  coarse budget, expansion; reference ``dsa_attention.py:3069-3542,3328-3384,4079-4217``),
  pinned by hand-written layouts and expansions and by ``F.avg_pool2d``;
* ``attention.sparse_attention_bwd``: explicit backward formulas of the reference kernel
  (reference ``easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py:534-743``),
  cross-checked against autograd on the forward restatement.

How each function is pinned (tests/test_oracle.py): brute-force pure-Python loops on tiny
shapes, closed forms (w = 1, Hi = 1 reduces to relu(scale q k^T)), the reference tests'
known-answer cases (tests/golden/), torch's own scaled_dot_product_attention for the dense
special case (kv_positions = arange), and exact backward invariants. No function of this
oracle is left "parity unpinned".
"""
