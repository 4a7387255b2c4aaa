"""Child process of test_zz_no_alloc.py: device free memory around a process's first calls
of the workspace dense forward and of the allocation-free one. Prints two byte counts: the
drop over a second workspace call (its code already loaded), then the drop over the first
allocation-free call (which brings the scratch array onto the device)."""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from geoweave_amd import _lib, workloads  # noqa: E402


def main():
    lib = _lib.load()
    q, k, v = (x.cuda() for x in workloads.attention_inputs(2, 1, torch.bfloat16, seed=71))
    B, T, H, D = q.shape
    S, K = k.shape[1], 512
    pos = workloads.distinct_positions(1, T, S, K, seed=72).cuda()
    o = torch.empty_like(q)
    lse = torch.empty(B, T, H, device="cuda")
    args = [_lib.dtype_code(q.dtype), q.data_ptr(), _lib.strides3(*q.stride()[:3]), k.data_ptr(),
            _lib.strides3(*k.stride()[:3]), v.data_ptr(), _lib.strides3(*v.stride()[:3]), pos.data_ptr(),
            pos.stride(0), pos.stride(1), o.data_ptr(), _lib.strides3(*o.stride()[:3]), lse.data_ptr(), None,
            B, T, S, H, D, K, 0.125, None, 0, 0, 0, 0.0, None]
    nbytes = int(lib.gw_sparse_attn_fwd_dense_workspace_size(B, T, S, H, D, K, 0))
    ws = torch.empty(nbytes, device="cuda", dtype=torch.uint8)
    stream = _lib.stream_handle(q.device)
    _lib.check(lib.gw_sparse_attn_fwd_dense(*args, ws.data_ptr(), nbytes, stream), "gw_sparse_attn_fwd_dense")
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    _lib.check(lib.gw_sparse_attn_fwd_dense(*args, ws.data_ptr(), nbytes, stream), "gw_sparse_attn_fwd_dense")
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    _lib.check(lib.gw_sparse_attn_fwd_dense_noalloc(*args, stream), "gw_sparse_attn_fwd_dense_noalloc")
    torch.cuda.synchronize()
    free2 = torch.cuda.mem_get_info()[0]
    print(free0 - free1, free1 - free2, flush=True)


if __name__ == "__main__":
    main()
