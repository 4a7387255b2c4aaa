"""The documented reference-side binding (geoweave_amd.reference_binding.install) on a stand-in
of the reference's package tree (CPU only: imports, no kernel calls).

The stand-in mirrors the layout the reference's import statements need: the real package
``easyvolcap/utils/custom_indexer`` imports its two leaf modules from its ``__init__`` and
sets ``sparse_topk_indexer_inference_func = None`` (reference ``__init__.py:1-7``); the
modules ``streaming_kl_autograd`` and ``topk_support_autograd``, which the reference's
``indexer.py:8-9`` imports outside any ``try``, must keep resolving; the leaf modules this
build replaces raise if they are ever executed. The test then runs the reference's import
statements (``indexer.py:7-14``, ``dsa_attention.py:24-45``) and checks that every name is
this build's object.
"""
import sys
import textwrap

import pytest

STUBS = {
    "easyvolcap/__init__.py": "",
    "easyvolcap/utils/__init__.py": "",
    "easyvolcap/utils/dist_utils.py": """
        def get_rank():
            return 0

        def is_main_process():
            return True
    """,
    "easyvolcap/utils/custom_indexer/__init__.py": """
        from .indexer_kl_fused import sparse_indexer_kl_loss
        from .sparse_topk_indexer import sparse_topk_indexer_func
        sparse_topk_indexer_inference_func = None
    """,
    "easyvolcap/utils/custom_indexer/indexer_kl_fused.py": """
        raise ImportError("stand-in: the replaced KL module must not be executed")
    """,
    "easyvolcap/utils/custom_indexer/sparse_topk_indexer.py": """
        def sparse_topk_indexer_func(*args, **kwargs):
            raise RuntimeError("stand-in of the reference kernel")

        def _compute_scores_block_triton(*args, **kwargs):
            raise RuntimeError("stand-in")
    """,
    "easyvolcap/utils/custom_indexer/streaming_kl_autograd.py": """
        from .sparse_topk_indexer import _compute_scores_block_triton

        def streaming_kl_autograd_loss(*args, **kwargs):
            return "reference streaming KL"

        def _score_chunk_forward(*args, **kwargs):
            return None
    """,
    "easyvolcap/utils/custom_indexer/topk_support_autograd.py": """
        from .streaming_kl_autograd import _score_chunk_forward

        def topk_support_autograd_loss(*args, **kwargs):
            return "reference top-k support loss"
    """,
    "easyvolcap/utils/custom_flash_attn/__init__.py": "",
    "easyvolcap/utils/custom_flash_attn/sparse_index_flash_attn.py": """
        raise ImportError("stand-in: the replaced attention module must not be executed")
    """,
}

# The reference's import statements at its two call sites.
REFERENCE_IMPORTS = """
from easyvolcap.utils.dist_utils import get_rank, is_main_process
from easyvolcap.utils.custom_indexer.streaming_kl_autograd import streaming_kl_autograd_loss
from easyvolcap.utils.custom_indexer.topk_support_autograd import topk_support_autograd_loss
try:
    from easyvolcap.utils.custom_indexer import sparse_topk_indexer_func, sparse_topk_indexer_inference_func
except Exception:
    sparse_topk_indexer_func = None
    sparse_topk_indexer_inference_func = None
try:
    from easyvolcap.utils.custom_indexer.indexer_kl_fused import sparse_indexer_kl_loss
except Exception:
    sparse_indexer_kl_loss = None
try:
    from easyvolcap.utils.custom_flash_attn.sparse_index_flash_attn import (
        sparse_index_flash_attn_func,
        sparse_index_flash_attn_bhtd_func,
        sparse_index_flash_attn_value_gate_bhtd_func,
        dense_index_flash_attn_func,
        sparse_index_flash_attn_inference_func,
        sparse_index_flash_attn_inference_bhtd_func,
    )
except Exception:
    sparse_index_flash_attn_func = None
"""


@pytest.fixture
def stub_tree(tmp_path, monkeypatch):
    for rel, text in STUBS.items():
        path = tmp_path / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(textwrap.dedent(text))
    monkeypatch.syspath_prepend(str(tmp_path))
    yield tmp_path
    for name in [n for n in sys.modules if n == "easyvolcap" or n.startswith("easyvolcap.")]:
        del sys.modules[name]


def test_install_binds_every_reference_name(stub_tree):
    from geoweave_amd import reference_binding
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as gw_attn
    from geoweave_amd.custom_indexer import indexer_kl_fused as gw_kl
    from geoweave_amd.custom_indexer import sparse_topk_indexer as gw_sti

    pkg = reference_binding.install()
    assert pkg.__file__.startswith(str(stub_tree)), "the reference package itself stays in place"
    ns = {}
    exec(REFERENCE_IMPORTS, ns)
    assert ns["streaming_kl_autograd_loss"]() == "reference streaming KL"
    assert ns["topk_support_autograd_loss"]() == "reference top-k support loss"
    assert ns["sparse_topk_indexer_func"] is gw_sti.sparse_topk_indexer_func
    assert ns["sparse_topk_indexer_inference_func"] is gw_sti.sparse_topk_indexer_inference_func
    assert ns["sparse_indexer_kl_loss"] is gw_kl.sparse_indexer_kl_loss
    for name in ("sparse_index_flash_attn_func", "sparse_index_flash_attn_bhtd_func",
                 "dense_index_flash_attn_func", "sparse_index_flash_attn_inference_func",
                 "sparse_index_flash_attn_inference_bhtd_func"):
        assert ns[name] is getattr(gw_attn, name), name
    assert ns["sparse_index_flash_attn_value_gate_bhtd_func"] is None  # the caller's own fallback
    # module-attribute access and `import ... as` forms resolve to the same objects
    import easyvolcap.utils.custom_flash_attn.sparse_index_flash_attn as m
    import easyvolcap.utils.custom_indexer as ci
    assert m is gw_attn and ci.indexer_kl_fused is gw_kl
    assert ci.sparse_topk_indexer_func is gw_sti.sparse_topk_indexer_func


def test_without_install_the_stand_in_fails_as_the_reference_would(stub_tree):
    # Control: the stand-in's replaced leaves really raise, so the test above proves they
    # were never executed.
    ns = {}
    with pytest.raises(ImportError):
        exec("import easyvolcap.utils.custom_indexer", ns)
