"""Routing of the masked dense passes around the limits of their 32-bit load offsets (CPU:
only the host-side checks run). A K token stride of 2^23 elements or more, or S beyond
2^25 - 64, must send the forward and the backward to the gather/CSR paths, which take any
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
    assert sifa.DENSE_MAX_S == (1 << 25) - 64 and sifa.DENSE_MAX_K_ROW_STRIDE == 1 << 23


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
