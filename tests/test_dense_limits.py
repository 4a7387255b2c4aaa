"""Routing of the masked dense passes around the limits of their 32-bit load offsets (CPU:
only the host-side checks run). A K token stride of 2^23 elements or more, or S beyond
2^25 - 128, must send the forward and the backward to the gather/CSR paths, which take any
stride; ordinary layer shapes, strided views of a packed qkv tensor included, stay dense."""
import torch

from geoweave_amd.custom_flash_attn import _backward, sparse_index_flash_attn as sifa


def _view(t, h, d, token_stride, layout="bthd"):
    # a [1, t, h, d] (or [1, h, t, d]) tensor with the given token stride, without storage (the
    # checks read strides and shapes only)
    if layout == "bthd":
        return torch.empty_strided((1, t, h, d), (t * token_stride, token_stride, d, 1), device="meta",
                                   dtype=torch.bfloat16)
    return torch.empty_strided((1, h, t, d), (t * token_stride, d, token_stride, 1), device="meta",
                               dtype=torch.bfloat16)


def test_forward_dense_fits_layer_shapes_and_packed_qkv():
    assert sifa._dense_fits(_view(43968, 16, 64, 16 * 64), "bthd", 43968)
    assert sifa._dense_fits(_view(43968, 16, 64, 3 * 16 * 64), "bthd", 43968)  # packed q, k, v rows
    assert sifa._dense_fits(_view(43968, 16, 64, 16 * 64, "bhtd"), "bhtd", 43968)


def test_forward_dense_refuses_huge_strides_and_lengths():
    assert not sifa._dense_fits(_view(8, 1, 64, sifa.DENSE_MAX_K_ROW_STRIDE), "bthd", 8)
    assert sifa._dense_fits(_view(8, 1, 64, sifa.DENSE_MAX_K_ROW_STRIDE - 8), "bthd", 8)
    assert not sifa._dense_fits(_view(8, 1, 64, 64), "bthd", sifa.DENSE_MAX_S + 1)
    assert sifa.DENSE_MAX_S == (1 << 25) - 128 and sifa.DENSE_MAX_K_ROW_STRIDE == 1 << 23


def test_backward_dense_fits():
    q = _view(32976, 16, 64, 1024)
    assert _backward._dense_fits(q, q, q, q, "bthd")
    big = _view(8, 1, 64, _backward.DENSE_MAX_ROW_STRIDE)
    small = _view(8, 1, 64, 64)
    for i in range(4):
        args = [small] * 4
        args[i] = big
        assert not _backward._dense_fits(*args, "bthd")
    long_q = _view(_backward.DENSE_MAX_LEN + 1, 1, 64, 64)
    assert not _backward._dense_fits(long_q, small, small, long_q, "bthd")


def _bwd_dense_rc(T, S):
    """Return code of gw_sparse_attn_bwd_dense for lengths T, S with fake (aligned, never
    dereferenced) pointers and no workspace: the length limits are checked before the
    workspace, so UNSUPPORTED (2) means refused on length, INVALID (1) means past it."""
    import ctypes

    from geoweave_amd import _lib

    lib = _lib.load()
    s3 = _lib.strides3(1024 * 64, 1024, 64)
    route = ctypes.c_void_p(16)
    return lib.gw_sparse_attn_bwd_dense(0, 16, s3, 16, s3, 16, s3, 16, 1, 1, 16, s3, 16, s3, 16, 16, s3, 16, s3, 16,
                                        s3, 1, T, S, 16, 64, 1, 0.125, route, None, 0, None)


def _fwd_dense_rc(T, S):
    """gw_sparse_attn_fwd_dense's return code, as _bwd_dense_rc."""
    from geoweave_amd import _lib

    lib = _lib.load()
    s3 = _lib.strides3(1024 * 64, 1024, 64)
    return lib.gw_sparse_attn_fwd_dense(0, 16, s3, 16, s3, 16, s3, 16, 1, 1, 16, s3, 16, None, 1, T, S, 16, 64, 1,
                                        0.125, None, 0, 0, 0, 0.0, None, None, 0, None)


def test_length_limits_match_the_kernels():
    # Whatever the Python routing keeps on the dense passes, the C entry points accept (past
    # the length checks: INVALID, 1, for the missing workspace); what they refuse
    # (UNSUPPORTED, 2) the routing sends to the gather/CSR paths. Backward: T padded to 256
    # and S to 128 below 2^25 and at most 65535 query blocks; forward: S padded to 128 below
    # 2^25, same query blocks. T = 2^25 - 128 passed the old routing and then failed.
    small = _view(8, 1, 64, 64)
    tmax = _backward.DENSE_MAX_T
    assert tmax == sifa.DENSE_MAX_T == 65528 * 32 and _backward.DENSE_MAX_LEN == (1 << 25) - 256
    lens = [8, tmax, tmax + 1, (1 << 25) - 256, (1 << 25) - 255, (1 << 25) - 128, (1 << 25) - 64, (1 << 25) - 63]
    for t in lens:
        for s_len in lens:
            tq, tk = _view(t, 1, 64, 64), _view(s_len, 1, 64, 64)
            rc = _bwd_dense_rc(t, s_len)
            assert rc in (1, 2)
            if _backward._dense_fits(tq, tk, tk, tq, "bthd"):
                assert rc == 1, (t, s_len)
            rc = _fwd_dense_rc(t, s_len)
            assert rc in (1, 2)
            if sifa._dense_fits(small, "bthd", s_len, t):
                assert rc == 1, (t, s_len)
    long_q = _view((1 << 25) - 128, 1, 64, 64)
    assert not _backward._dense_fits(long_q, small, small, long_q, "bthd")
    assert _bwd_dense_rc((1 << 25) - 128, 8) == 2
    at_lim = _view(tmax, 1, 64, 64)
    assert _backward._dense_fits(at_lim, small, small, at_lim, "bthd")
