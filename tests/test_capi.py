"""CPU checks of the C ABI: the library loads, exports every declared symbol, and rejects
bad arguments with an error code and message before touching the GPU."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from geoweave_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "geoweave_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gw_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared, "no gw_* functions found in the header"
    assert sorted(_lib.exported_names()) == declared


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.gw_abi_version() == 105


def test_one_hip_runtime_in_process():
    _lib.load()
    maps = Path("/proc/self/maps").read_text().splitlines()
    runtimes = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes


def _attn_call(**over):
    lib = _lib.load()
    s = _lib.strides3(1024, 1024, 64)
    args = dict(dtype=0, q=16, k=16, v=16, pos=16, o=16, lse=None, attn=None,
                B=1, T=4, S=4, H=16, D=64, K=4, scale=0.125, ws=None, ws_bytes=0)
    args.update(over)
    return lib.gw_sparse_attn_fwd(
        args["dtype"], args["q"], s, args["k"], s, args["v"], s, args["pos"], 16, 4,
        args["o"], s, args["lse"], args["attn"], args["B"], args["T"], args["S"], args["H"],
        args["D"], args["K"], args["scale"], args["ws"], args["ws_bytes"], None)


def test_attn_fwd_rejects_bad_arguments_without_gpu():
    lib = _lib.load()
    assert _attn_call(dtype=7) == 1
    assert b"dtype" in lib.gw_last_error()
    assert _attn_call(D=32) == 2  # unsupported head dim
    assert b"head dim" in lib.gw_last_error()
    assert _attn_call(q=None) == 1
    assert _attn_call(q=18) == 1  # misaligned
    assert b"aligned" in lib.gw_last_error()
    assert _attn_call(attn=16) == 1  # attn_sum without workspace
    assert b"workspace" in lib.gw_last_error()
    assert _attn_call(B=0) == 0  # empty batch is a no-op
    assert lib.gw_sparse_attn_fwd_workspace_size(1, 10, 16, 8, 1) == 10 * 8 * 16 * 4
    assert lib.gw_sparse_attn_fwd_workspace_size(1, 10, 16, 8, 0) == 0


def test_check_raises_runtime_error_with_message():
    lib = _lib.load()
    rc = _attn_call(dtype=9)
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.check(rc, "gw_sparse_attn_fwd")


def test_python_preconditions_match_reference_errors():
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as m

    q = torch.zeros(1, 4, 2, 64, dtype=torch.float32)
    pos = torch.zeros(1, 4, 3, dtype=torch.int32)
    with pytest.raises(TypeError, match="fp16 and bf16"):
        m._flash_attn_forward(q, q, q, pos)
    qb = q.bfloat16()
    with pytest.raises(ValueError, match="head dimensions up to 128"):
        big = torch.zeros(1, 4, 2, 192, dtype=torch.bfloat16)
        m._flash_attn_forward(big, big, big, pos)
    with pytest.raises(ValueError, match="GPU tensors"):
        m._flash_attn_forward(qb, qb, qb, pos)


def test_dropin_modules_export_every_name_the_reference_callers_import():
    # easyvolcap/official_vggt/layers/dsa_attention.py:29-45 imports these six names in one
    # try block and :24-27 the KL loss; easyvolcap/official_vggt/layers/indexer.py:10-14
    # imports the two top-k entries.
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as m
    from geoweave_amd import custom_indexer

    for name in ("sparse_index_flash_attn_func", "sparse_index_flash_attn_bhtd_func",
                 "sparse_index_flash_attn_value_gate_bhtd_func", "dense_index_flash_attn_func",
                 "sparse_index_flash_attn_inference_func", "sparse_index_flash_attn_inference_bhtd_func"):
        assert hasattr(m, name), name
    assert m.sparse_index_flash_attn_value_gate_bhtd_func is None
    assert callable(custom_indexer.sparse_topk_indexer_func)
    assert callable(custom_indexer.sparse_topk_indexer_inference_func)
    assert callable(custom_indexer.sparse_indexer_kl_loss)


def test_kl_loss_rejects_cpu_tensors_and_shape_mismatch():
    # The reference falls back to a torch formula here (indexer_kl_fused.py:286-295); this
    # package has no CPU path, so it raises instead.
    from geoweave_amd.custom_indexer import sparse_indexer_kl_loss

    a = torch.rand(1, 3, 8)
    with pytest.raises(ValueError, match="GPU tensors"):
        sparse_indexer_kl_loss(a, torch.randn(1, 3, 8))
    with pytest.raises(ValueError, match="must be equal"):
        sparse_indexer_kl_loss(a, torch.randn(1, 3, 9))
    empty = torch.zeros(1, 0, 8)
    assert float(sparse_indexer_kl_loss(empty, empty)) == 0.0


def test_reuse_topk_group_and_layer_parsers_follow_the_reference_syntax():
    # easyvolcap/official_vggt/models/aggregator.py:267-292 and :327-362
    from geoweave_amd.aggregator import parse_indexer_layers, parse_reuse_topk_groups

    assert parse_indexer_layers("9-19") == set(range(9, 20))
    assert parse_indexer_layers("1,3, 5-7") == {1, 3, 5, 6, 7}
    assert parse_indexer_layers("all") is None and parse_indexer_layers("*") is None
    assert parse_indexer_layers("") == set() and parse_indexer_layers(None) is None
    assert parse_indexer_layers([2, "4"]) == {2, 4}
    assert parse_reuse_topk_groups("9:10,11") == {10: 9}  # "11" alone names no reuse
    assert parse_reuse_topk_groups("9:10-12") == {10: 9, 11: 9, 12: 9}
    assert parse_reuse_topk_groups("9-12") == {10: 9, 11: 9, 12: 9}
    assert parse_reuse_topk_groups("12-9") == {10: 9, 11: 9, 12: 9}
    assert parse_reuse_topk_groups(["9:9-10", "14-15"]) == {10: 9, 15: 14}
    assert parse_reuse_topk_groups("") == {} and parse_reuse_topk_groups(None) is None


def test_special_tokens_first_view_uses_slot_zero():
    # aggregator.py:723-746
    from geoweave_amd.aggregator import slice_expand_and_flatten

    tok = torch.arange(2 * 3 * 4, dtype=torch.float32).view(1, 2, 3, 4)
    out = slice_expand_and_flatten(tok, 2, 3).view(2, 3, 3, 4)
    for b in range(2):
        assert torch.equal(out[b, 0], tok[0, 0])
        assert torch.equal(out[b, 1], tok[0, 1]) and torch.equal(out[b, 2], tok[0, 1])


def _dense_call(**over):
    lib = _lib.load()
    s = _lib.strides3(1024, 1024, 64)
    args = dict(dtype=0, q=16, k=16, v=16, pos=16, o=16, lse=16, attn=None, B=1, T=4, S=4, H=16, D=64, K=4,
                scale=0.125, logits=None, row_loss=None, ws=None, ws_bytes=0)
    args.update(over)
    return lib.gw_sparse_attn_fwd_dense(
        args["dtype"], args["q"], s, args["k"], s, args["v"], s, args["pos"], 16, 4,
        args["o"], s, args["lse"], args["attn"], args["B"], args["T"], args["S"], args["H"], args["D"],
        args["K"], args["scale"], args["logits"], 2, 4, 1, 1e-6, args["row_loss"], args["ws"], args["ws_bytes"], None)


def test_dense_fwd_workspace_and_argument_checks_without_gpu():
    lib = _lib.load()
    # mask: 4 sub-tiles of 32 keys (S padded to 128) x 256 queries (1 block padded to the 8 of
    # a workgroup) x 4 B = 4096; block flags 4 B -> 4352; non-finite flag per batch element
    # 4 B -> 4608; |V| column maxima 16 heads x 64 x 4 B -> 8704; V^T 16 heads x 64 x 128
    # keys x 2 B
    base = 4608 + 16 * 64 * 4 + 16 * 64 * 128 * 2
    assert lib.gw_sparse_attn_fwd_dense_workspace_size(1, 4, 4, 16, 64, 4, 0) == base
    # + the selected scores for attn_sum: T x (K rounded up to 8, + 8) x H x 4 B
    assert lib.gw_sparse_attn_fwd_dense_workspace_size(1, 4, 4, 16, 64, 4, 1) == base + 4 * 16 * 16 * 4
    assert lib.gw_sparse_attn_fwd_dense_workspace_size(1, 4, 4, 16, 128, 4, 0) == 0
    assert _dense_call(D=128) == 2
    assert b"head dim" in lib.gw_last_error()
    assert _dense_call(attn=16, K=2048) == 2
    assert b"K <= 1024" in lib.gw_last_error()
    assert _dense_call(scale=-0.125) == 2 and _dense_call(scale=0.0) == 2
    assert b"positive finite softmax scale" in lib.gw_last_error()
    assert _dense_call(dtype=7) == 1
    assert _dense_call() == 1
    assert b"workspace" in lib.gw_last_error()
    assert _dense_call(logits=16, row_loss=16, ws=4096, ws_bytes=1 << 20) == 1
    assert b"needs attn_sum" in lib.gw_last_error()
    assert _dense_call(attn=16, lse=None, ws=4096, ws_bytes=1 << 20) == 1
    assert b"lse" in lib.gw_last_error()
    assert _dense_call(q=18, ws=4096, ws_bytes=1 << 20) == 1
    assert _dense_call(B=0) == 0  # nothing to do


def _topk_call(**over):
    lib = _lib.load()
    args = dict(dtype=2, q=16, k=16, w=16, mask=None, B=1, T=4, S=4, Hi=4, Di=64, topk=2, scale=0.125,
                flags=0, idx=16, sc=16, ws=None, ws_bytes=0)
    args.update(over)
    return lib.gw_indexer_topk_fwd(args["dtype"], args["q"], args["k"], args["w"], args["mask"], args["B"],
                                   args["T"], args["S"], args["Hi"], args["Di"], args["topk"], args["scale"],
                                   args["flags"], args["idx"], args["sc"], args["ws"], args["ws_bytes"], None)


def test_indexer_fwd_dtype_rules_without_gpu():
    # fp32 is a valid indexer dtype (the reference computes in q.dtype,
    # sparse_topk_indexer.py:1293); 8 fp32 heads are not built; other codes are invalid.
    lib = _lib.load()
    assert _topk_call(dtype=3) == 1 and b"dtype" in lib.gw_last_error()
    assert _topk_call(dtype=2, Hi=8) == 2 and b"fp32" in lib.gw_last_error()
    for dt in (0, 1, 2):
        assert _topk_call(dtype=dt) == 1 and b"workspace" in lib.gw_last_error()  # passes the dtype check
    assert _topk_call(dtype=2, B=0) == 0


def test_indexer_dtype_codes_in_python():
    assert _lib.dtype_code(torch.float32, allow_fp32=True) == _lib.GW_DTYPE_FP32
    with pytest.raises(TypeError, match="bfloat16 or float16"):
        _lib.dtype_code(torch.float32)
    with pytest.raises(TypeError):
        _lib.dtype_code(torch.float64, allow_fp32=True)
