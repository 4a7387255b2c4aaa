"""GPU checks of the key-major (CSR) table built by ``gw_kv_csr_build``.

The buffer is read back and compared field by field with a numpy construction from the
definition: entries of key ``b*S + s`` are the ``(t, j)`` with ``pos[b, t, j] == s`` in
``(t, j)`` order, positions outside ``[0, S)`` are dropped, a key's entries are split into
work items of at most 2048, and keys split over several items get partial-sum slots.
Cases cover one and several radix passes, hub keys longer than a work item, invalid
positions, tails that do not fill a 2048-entry tile, empty keys and an all-invalid table.
"""
import numpy as np
import pytest
import torch

from geoweave_amd import _csr

pytestmark = pytest.mark.gpu

CHUNK = 2048  # entries per work item


def _layout(B, T, S, K):
    """Byte offsets of the buffer's regions: each region starts on a 256-byte boundary."""
    nk, ne = B * S, B * T * K
    o = 0
    out = {}
    max_items = nk + (ne + CHUNK - 1) // CHUNK
    for name, nbytes in (("header", 16), ("count", nk * 4), ("off", (nk + 1) * 4),
                         ("item_off", (nk + 1) * 4), ("part_off", (nk + 1) * 4),
                         ("item_key", max_items * 4), ("entries", ne * 8)):
        out[name] = o
        o = (o + nbytes + 255) // 256 * 256
    return out


def _expected(pos, S):
    B, T, K = pos.shape
    nk = B * S
    b, t, j = np.meshgrid(np.arange(B), np.arange(T), np.arange(K), indexing="ij")
    s = pos.reshape(-1)
    ok = (s >= 0) & (s < S)
    key = (b.reshape(-1) * S + s)[ok]
    order = np.argsort(key, kind="stable")  # row-major input order => (t, j) within a key
    entries = np.stack([t.reshape(-1)[ok][order], j.reshape(-1)[ok][order]], axis=1)
    count = np.bincount(key, minlength=nk)
    off = np.concatenate([[0], np.cumsum(count)])
    items = np.maximum(1, (count + CHUNK - 1) // CHUNK)
    item_off = np.concatenate([[0], np.cumsum(items)])
    part_off = np.concatenate([[0], np.cumsum(np.where(items > 1, items, 0))])
    item_key = np.repeat(np.arange(nk), items)
    return dict(off=off, item_off=item_off, part_off=part_off, item_key=item_key, entries=entries,
                header=(int(item_off[-1]), int(part_off[-1])))


def _build(pos, S):
    csr, nbytes = _csr.build(pos.cuda(), S, cache=False)
    torch.cuda.synchronize()
    return csr.cpu().numpy()


def _field(buf, at, n, dtype=np.int32):
    return np.frombuffer(buf[at:at + n * np.dtype(dtype).itemsize].tobytes(), dtype=dtype)


def _check(pos, S):
    B, T, K = pos.shape
    want = _expected(pos.numpy(), S)
    buf = _build(pos, S)
    L = _layout(B, T, S, K)
    nk = B * S
    hdr = _field(buf, L["header"], 2)
    assert tuple(hdr) == want["header"]
    np.testing.assert_array_equal(_field(buf, L["off"], nk + 1), want["off"])
    np.testing.assert_array_equal(_field(buf, L["item_off"], nk + 1), want["item_off"])
    np.testing.assert_array_equal(_field(buf, L["part_off"], nk + 1), want["part_off"])
    np.testing.assert_array_equal(_field(buf, L["item_key"], hdr[0]), want["item_key"])
    n_valid = int(want["off"][-1])
    got = _field(buf, L["entries"], 2 * n_valid).reshape(-1, 2)
    np.testing.assert_array_equal(got, want["entries"])


@pytest.mark.parametrize("B,T,S,K,seed", [
    (1, 40, 50, 8, 0),        # one pass (keys 0..50 < 64)
    (1, 300, 700, 48, 1),     # two passes, ragged tail tile
    (2, 700, 2500, 64, 2),    # B = 2, three passes
    (1, 5000, 5000, 256, 3),  # several full tiles
])
def test_csr_matches_definition(gpu_device, B, T, S, K, seed):
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(0, S, (B, T, K), generator=g, dtype=torch.int32)
    print(f"[csr] B={B} T={T} S={S} K={K}", flush=True)
    _check(pos, S)


def test_csr_hub_keys_and_invalid_positions(gpu_device):
    B, T, S, K = 2, 3000, 3000, 64
    g = torch.Generator().manual_seed(11)
    pos = torch.randint(0, S, (B, T, K), generator=g, dtype=torch.int32)
    pos[0, :, 0] = 7           # key chosen by every query: 3000 > one work item
    pos[1, :, :3] = 2999       # 9000 entries on the last key of batch 1
    pos[0, 10, :] = -1         # fully masked row
    pos[1, 20:40, 5:] = S      # out of range -> dropped
    pos[1, 50, 1] = -7
    _check(pos, S)


def test_csr_empty_keys_and_all_invalid(gpu_device):
    # Most keys are never chosen (long runs of empty keys between the chosen ones).
    g = torch.Generator().manual_seed(12)
    pos = (torch.randint(0, 20, (1, 100, 16), generator=g, dtype=torch.int32) * 997) % 20000
    _check(pos, 20000)
    # No valid entry at all.
    _check(torch.full((1, 30, 8), -1, dtype=torch.int32), 500)


def test_csr_is_deterministic(gpu_device):
    g = torch.Generator().manual_seed(13)
    pos = torch.randint(0, 4000, (1, 4000, 128), generator=g, dtype=torch.int32)
    pos[0, :, :4] = 5
    a = _build(pos, 4000)
    b = _build(pos, 4000)
    L = _layout(1, 4000, 4000, 128)
    n_items = int(_field(a, L["header"], 1)[0])
    for name, n in (("header", 2), ("off", 4001), ("item_off", 4001), ("part_off", 4001),
                    ("item_key", n_items), ("entries", 2 * 4000 * 128)):
        np.testing.assert_array_equal(_field(a, L[name], n), _field(b, L[name], n))


def test_only_the_table_stays_allocated(gpu_device):
    # The radix sort's ping-pong buffers (16 bytes per entry) are a transient workspace:
    # after a C4-size build (B = 2, N = 32,976, K = 1,024) only the table stays allocated.
    from geoweave_amd import _lib, workloads

    B, n, K = 2, 32976, 1024
    pos = workloads.distinct_positions(B, n, n, K, seed=3).cuda()
    lib = _lib.load()
    table = int(lib.gw_kv_csr_size(B, n, n, K))
    scratch = int(lib.gw_kv_csr_build_workspace_size(B, n, n, K))
    assert scratch >= 16 * B * n * K
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    csr, nbytes = _csr.build(pos, n, cache=False)
    torch.cuda.synchronize()
    kept = torch.cuda.memory_allocated() - before
    assert nbytes == table and kept <= table + (2 << 20), f"{kept} bytes kept for a {table}-byte table"
    print(f"[csr] table {table / 2**30:.2f} GiB kept, build workspace {scratch / 2**30:.2f} GiB released",
          flush=True)
