"""GPU check of the allocation-free dense forward (gw_sparse_attn_fwd_dense_noalloc) through
the C ABI: two calls in a row (the second smaller, so stale contents of the shared scratch
from the first call would show), each against gw_sparse_attn_fwd_dense with a caller
workspace on the same inputs. Both run the same kernels, so o, lse and attn_sum must be
bit-identical; the first case is also checked against the fp32 oracle at the attention
tolerance. A call beyond the scratch capacity is refused on the host. The entry point is
also captured into a graph (its first call on the device inside the capture) and replayed,
and a fresh process shows that the scratch array takes device memory only from the first
allocation-free call on, not when the library's other kernels run.
"""
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from geoweave_amd import _lib, workloads
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _args(q, k, v, pos, o, lse, attn, scale):
    B, T, H, D = q.shape
    S, K = k.shape[1], pos.shape[-1]
    return [_lib.dtype_code(q.dtype), q.data_ptr(), _lib.strides3(*q.stride()[:3]),
            k.data_ptr(), _lib.strides3(*k.stride()[:3]), v.data_ptr(), _lib.strides3(*v.stride()[:3]),
            pos.data_ptr(), pos.stride(0), pos.stride(1), o.data_ptr(), _lib.strides3(*o.stride()[:3]),
            lse.data_ptr(), _lib.ptr(attn), B, T, S, H, D, K, float(scale), None, 0, 0, 0, 0.0, None]


def _both(q, k, v, pos, with_attn, scale=0.125):
    lib = _lib.load()
    dev = q.device
    B, T, H, D = q.shape
    S, K = k.shape[1], pos.shape[-1]
    outs = []
    for noalloc in (True, False):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((B, T, H), float("nan"), device=dev)
        attn = torch.full((B, T, K), float("nan"), device=dev) if with_attn else None
        args = _args(q, k, v, pos, o, lse, attn, scale)
        stream = _lib.stream_handle(dev)
        if noalloc:
            rc = lib.gw_sparse_attn_fwd_dense_noalloc(*args, stream)
            _lib.check(rc, "gw_sparse_attn_fwd_dense_noalloc")
        else:
            nbytes = int(lib.gw_sparse_attn_fwd_dense_workspace_size(B, T, S, H, D, K, int(with_attn)))
            ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
            rc = lib.gw_sparse_attn_fwd_dense(*args, ws.data_ptr(), nbytes, stream)
            _lib.check(rc, "gw_sparse_attn_fwd_dense")
        torch.cuda.synchronize()
        outs.append((o.cpu(), lse.cpu(), None if attn is None else attn.cpu()))
    return outs


def test_noalloc_under_graph_capture_allocates_nothing(gpu_device):
    # The callers this entry point is for capture it into a graph. It runs first in this
    # file and nothing else calls it, so the process's first call on the device (the scratch
    # address lookup included) happens inside the capture. Every replay, with eager work
    # between replays, equals the workspace entry's eager result. Afterwards an eager call
    # (its kernels' code already loaded) leaves the device's free memory unchanged.
    lib = _lib.load()
    q, k, v = workloads.attention_inputs(2, 1, torch.bfloat16, seed=61)
    pos = workloads.distinct_positions(1, q.shape[1], k.shape[1], 512, seed=62)
    qd, kd, vd, pd = (x.cuda() for x in (q, k, v, pos))
    B, T, H, _ = q.shape
    o = torch.full_like(qd, float("nan"))
    lse = torch.full((B, T, H), float("nan"), device="cuda")
    args = _args(qd, kd, vd, pd, o, lse, None, 0.125)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=side):
        rc = lib.gw_sparse_attn_fwd_dense_noalloc(*args, _lib.stream_handle(qd.device))
    torch.cuda.synchronize()
    assert rc == 0, lib.gw_last_error()
    _, (o_w, l_w, _) = _both(qd, kd, vd, pd, False)
    for replay in range(3):
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        print(f"[noalloc] graph replay {replay}", flush=True)
        assert torch.equal(o.cpu(), o_w) and torch.equal(lse.cpu(), l_w)
    free0 = torch.cuda.mem_get_info()[0]
    rc = lib.gw_sparse_attn_fwd_dense_noalloc(*args, _lib.stream_handle(qd.device))
    torch.cuda.synchronize()
    assert rc == 0 and torch.cuda.mem_get_info()[0] == free0


@pytest.mark.parametrize("with_attn", [False, True])
def test_noalloc_equals_the_workspace_entry_on_two_calls(gpu_device, with_attn):
    lib = _lib.load()
    cap = int(lib.gw_sparse_attn_fwd_dense_noalloc_capacity())
    assert cap == 64 << 20
    # call 1: two views of the layer (N = 2,748, K = 1,024; with attn_sum K = 256);
    # call 2: a smaller ragged cross-attention shape with a repeated position
    K1 = 256 if with_attn else 1024
    q1, k1, v1 = workloads.attention_inputs(2, 1, torch.bfloat16, seed=51)
    pos1 = workloads.distinct_positions(1, q1.shape[1], k1.shape[1], K1, seed=52)
    g = torch.Generator().manual_seed(53)
    q2 = torch.randn(2, 300, 16, 64, generator=g).bfloat16()
    k2 = torch.randn(2, 700, 16, 64, generator=g).bfloat16()
    v2 = torch.randn(2, 700, 16, 64, generator=g).bfloat16()
    pos2 = workloads.random_positions(2, 300, 700, 100, seed=54, invalid_fraction=0.3)
    pos2[1, 40, :3] = 9
    for case, (q, k, v, pos) in enumerate(((q1, k1, v1, pos1), (q2, k2, v2, pos2))):
        print(f"[noalloc] call {case + 1} with_attn={with_attn} T={q.shape[1]} S={k.shape[1]} K={pos.shape[-1]}",
              flush=True)
        qd, kd, vd, pd = (x.cuda() for x in (q, k, v, pos))
        (o_n, l_n, a_n), (o_w, l_w, a_w) = _both(qd, kd, vd, pd, with_attn)
        assert torch.equal(o_n, o_w) and torch.equal(l_n, l_w)
        if with_attn:
            assert torch.equal(a_n, a_w)
        if case == 0:
            rows = torch.randperm(q.shape[1], generator=g)[:96]
            ro, ra, rl = oatt.sparse_attention(q[:, rows], k, v, pos[:, rows], 0.125)
            torch.testing.assert_close(o_n[:, rows].float(), ro, atol=2e-2, rtol=2e-2)
            torch.testing.assert_close(l_n[:, rows], rl, atol=1e-4, rtol=1e-4)
            if with_attn:
                torch.testing.assert_close(a_n[:, rows], ra, atol=1e-4, rtol=1e-3)


def test_noalloc_refuses_calls_beyond_its_scratch(gpu_device):
    lib = _lib.load()
    B, T, S, H, D, K = 1, 21984, 21984, 16, 64, 1024  # 16 views: ~150 MB of workspace
    assert lib.gw_sparse_attn_fwd_dense_workspace_size(B, T, S, H, D, K, 0) > (64 << 20)
    q = torch.empty(B, T, H, D, device="cuda", dtype=torch.bfloat16)
    pos = torch.empty(B, T, K, device="cuda", dtype=torch.int32)
    o = torch.empty_like(q)
    lse = torch.empty(B, T, H, device="cuda")
    rc = lib.gw_sparse_attn_fwd_dense_noalloc(*_args(q, q, q, pos, o, lse, None, 0.125), _lib.stream_handle(q.device))
    assert rc == 2  # GW_ERR_UNSUPPORTED
    assert b"allocation-free" in lib.gw_last_error()


def test_scratch_is_resident_only_from_the_first_call(gpu_device):
    # A fresh process (this one may have called the entry point already): a second workspace
    # call leaves the device's free memory as it was (within 8 MiB of runtime bookkeeping),
    # the first allocation-free call takes the 64 MiB array.
    child = Path(__file__).resolve().parent / "noalloc_residency_child.py"
    print("[noalloc] residency child process", flush=True)
    res = subprocess.run([sys.executable, str(child)], capture_output=True, text=True, timeout=240)
    assert res.returncode == 0, res.stderr[-2000:]
    before, first = (int(x) for x in res.stdout.split()[-2:])
    print(f"[noalloc] free-memory drop: second workspace call {before} B, first allocation-free call {first} B")
    assert before < 8 << 20
    assert first >= 64 << 20
