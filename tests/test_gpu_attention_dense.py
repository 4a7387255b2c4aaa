"""GPU parity of the masked dense attention forward (gw_sparse_attn_fwd_dense) against the
fp32 CPU oracle and the gather kernel.

The dense pass computes every (query, key) product on the matrix cores and masks the keys a
query did not select; o and lse must equal the sparse attention's. Tolerance: 2e-2 abs/rel for
bf16/fp16 outputs (P enters the P·V product in fp16 against V scaled per column by a power of
two; the row sums add that fp16 operand in fp32), 1e-4 for lse. Cases: V columns far outside the fp16
range and far below it (the per-column scaling), odd head counts, a softmax scale other than
1/8, the layer's per-view shape in bf16 and fp16, ragged -1
padding with T and S not multiples of 32 or 64, cross attention (T != S), empty rows,
out-of-range and repeated positions (repeats go to the gather kernel inside the call, also
when the mask is built in several key chunks), scores with a large dynamic range rising along
the key order (the lazy maximum is raised and O rescaled on many tiles), key counts around
the 64- and 128-key tile boundaries, bhtd strides, determinism, and a full-size layer on
sampled rows.
"""
import contextlib

import pytest
import torch

from geoweave_amd import workloads
from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)


@contextlib.contextmanager
def _path(name):
    old = sifa.FORWARD_PATH
    sifa.FORWARD_PATH = name
    try:
        yield
    finally:
        sifa.FORWARD_PATH = old


def _run(q, k, v, pos, scale=None, layout="bthd", path="dense"):
    qd, kd, vd, pd = (x.cuda() for x in (q, k, v, pos))
    if layout == "bhtd":
        qd, kd, vd = (x.transpose(1, 2).contiguous() for x in (qd, kd, vd))
    with _path(path):
        o, attn, lse, _ = sifa._flash_attn_forward(qd, kd, vd, pd, softmax_scale=scale, return_attn=False,
                                                   q_layout=layout)
    torch.cuda.synchronize()
    assert attn is None
    if layout == "bhtd":
        o = o.transpose(1, 2)
    return o.float().cpu(), lse.cpu()


def _distinct_positions(B, T, S, K, seed):
    # Row t lists (off_t + j * step) mod S: distinct when gcd(step, S) = 1.
    g = torch.Generator().manual_seed(seed)
    step = 7919 if S % 7919 else 7907
    off = torch.randint(0, S, (B, T, 1), generator=g)
    j = torch.arange(K).view(1, 1, K)
    return ((off + j * step) % S).to(torch.int32).contiguous()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_one_view_layer_shape(gpu_device, dtype):
    q, k, v = workloads.attention_inputs(1, 1, dtype)
    n = q.shape[1]
    pos = workloads.random_positions(1, n, n, 1024, seed=21)
    print(f"[dense] one view N={n} dtype={dtype}", flush=True)
    o, lse = _run(q, k, v, pos)
    ro, _, rl = oatt.sparse_attention(q, k, v, pos)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)
    og, lg = _run(q, k, v, pos, path="gather")
    torch.testing.assert_close(o, og, **TOL)
    torch.testing.assert_close(lse, lg, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("B,T,S,H,K,inv", [(2, 300, 300, 4, 77, 0.5), (1, 5, 700, 2, 64, 0.0),
                                            (1, 100, 70, 16, 70, 0.3), (2, 257, 1000, 6, 200, 0.2)])
def test_ragged_and_cross_attention(gpu_device, B, T, S, H, K, inv):
    g = torch.Generator().manual_seed(T + S)
    q = torch.randn(B, T, H, 64, generator=g).bfloat16()
    k = torch.randn(B, S, H, 64, generator=g).bfloat16()
    v = torch.randn(B, S, H, 64, generator=g).bfloat16()
    pos = workloads.random_positions(B, T, S, K, seed=T, invalid_fraction=inv)
    print(f"[dense] B={B} T={T} S={S} H={H} K={K}", flush=True)
    o, lse = _run(q, k, v, pos, scale=0.1)
    ro, _, rl = oatt.sparse_attention(q, k, v, pos, 0.1)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)


def test_masking_and_repeated_positions(gpu_device):
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=200, seed=9)
    pos = workloads.random_positions(1, 200, 200, 13, seed=10)
    pos[0, 0, :] = -1          # no valid candidate: o = 0, lse = -inf
    pos[0, 1, 5:] = 200        # past the end: masked
    pos[0, 3, 0] = -5
    pos[0, 70, :] = 7          # one position listed 13 times: counted 13 times (gather kernel)
    pos[0, 150, 2] = pos[0, 150, 9]
    o, lse = _run(q, k, v, pos)
    ro, _, rl = oatt.sparse_attention(q, k, v, pos)
    assert torch.all(o[0, 0] == 0) and torch.isinf(lse[0, 0]).all() and (lse[0, 0] < 0).all()
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)
    # the repeated key dominates nothing: with one key listed 13 times the row is v[7]
    torch.testing.assert_close(o[0, 70], v[0, 7].float(), **TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_large_dynamic_range_rising_scores(gpu_device, dtype):
    # Scores grow along the key order by ~60 units of log2 over the keys, so the lazy
    # maximum of every row is raised on many tiles and O is rescaled each time.
    T, S, H, K = 96, 2048, 2, 512
    g = torch.Generator().manual_seed(5)
    q = (torch.ones(1, T, H, 64) + 0.1 * torch.randn(1, T, H, 64, generator=g))
    ramp = torch.linspace(-3.0, 3.0, S).view(1, S, 1, 1)
    k = ramp * torch.ones(1, S, H, 64) + 0.1 * torch.randn(1, S, H, 64, generator=g)
    v = torch.randn(1, S, H, 64, generator=g)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    pos = workloads.random_positions(1, T, S, K, seed=6)
    o, lse = _run(q, k, v, pos, scale=0.125)
    ro, _, rl = oatt.sparse_attention(q, k, v, pos, 0.125)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)


def test_bhtd_matches_bthd_and_is_deterministic(gpu_device):
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=512, seed=3)
    pos = workloads.random_positions(1, 512, 512, 200, seed=4)
    o1, l1 = _run(q, k, v, pos)
    o2, l2 = _run(q, k, v, pos, layout="bhtd")
    o3, l3 = _run(q, k, v, pos)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert torch.equal(o1, o3) and torch.equal(l1, l3)


@pytest.mark.parametrize("views", [16, 64])  # 64 views: N = 87,936, the C3 shape
def test_full_size_sampled_rows(gpu_device, views):
    q, k, v = workloads.attention_inputs(views, 1, torch.bfloat16)
    n = q.shape[1]
    pos = _distinct_positions(1, n, n, 1024, seed=views)
    print(f"[dense] full size N={n}", flush=True)
    o, lse = _run(q, k, v, pos)
    og, lg = _run(q, k, v, pos, path="gather")
    torch.testing.assert_close(o, og, **TOL)
    torch.testing.assert_close(lse, lg, atol=1e-4, rtol=1e-4)
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(1))[:128]
    ro, _, rl = oatt.sparse_attention(q[:, rows], k, v, pos[:, rows])
    torch.testing.assert_close(o[:, rows], ro, **TOL)
    torch.testing.assert_close(lse[:, rows], rl, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("S", [40000, 90000])
def test_repeated_position_in_an_upper_key_range(gpu_device, S):
    # The selection words come from one pass over the positions with 16 queries per workgroup
    # (S = 40,000) or from key chunks of 16,384 (S = 90,000: more sub-tiles than the LDS of one
    # pass holds); a repeat among the last keys flags its block like one among the first, and
    # the gather kernel computes that block.
    T, H, K = 80, 2, 256
    g = torch.Generator().manual_seed(31)
    q = torch.randn(1, T, H, 64, generator=g).bfloat16()
    k = torch.randn(1, S, H, 64, generator=g).bfloat16()
    v = torch.randn(1, S, H, 64, generator=g).bfloat16()
    pos = _distinct_positions(1, T, S, K, seed=32)
    pos[0, 40, 7] = S - 1
    pos[0, 40, 8] = S - 1      # block 1 (rows 32..63): repeat among the last keys
    pos[0, 75, :5] = S // 2    # block 2: five copies
    pos[0, 20, 3] = S - 2      # block 0: a key near the end
    print(f"[dense] repeated positions S={S}", flush=True)
    o, lse = _run(q, k, v, pos)
    ro, _, rl = oatt.sparse_attention(q, k, v, pos)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)


def _run_attn(q, k, v, pos, scale=None, path="dense", layout="bthd", kl=None):
    qd, kd, vd, pd = (x.cuda() for x in (q, k, v, pos))
    if layout == "bhtd":
        qd, kd, vd = (x.transpose(1, 2).contiguous() for x in (qd, kd, vd))
    extra = {}
    if kl is not None:
        extra = dict(kl_logits=kl.cuda(), kl_eps=1e-6,
                     kl_row_loss=torch.empty(q.shape[0] * q.shape[1], device="cuda", dtype=torch.float32))
    with _path(path):
        o, attn, lse, _ = sifa._flash_attn_forward(qd, kd, vd, pd, softmax_scale=scale, return_attn=True,
                                                   q_layout=layout, **extra)
    torch.cuda.synchronize()
    if layout == "bhtd":
        o = o.transpose(1, 2)
    loss = extra["kl_row_loss"].cpu() if kl is not None else None
    return o.float().cpu(), attn.cpu(), lse.cpu(), loss


@pytest.mark.parametrize("B,T,S,H,K,inv", [(1, 1374, 1374, 16, 1024, 0.0), (2, 300, 300, 4, 77, 0.5),
                                            (1, 257, 1000, 6, 200, 0.2), (1, 70, 70, 2, 64, 0.3)])
def test_attn_sum_matches_oracle(gpu_device, B, T, S, H, K, inv):
    # attn_sum from the slot-indexed scores and the sorted positions; o unchanged by it
    g = torch.Generator().manual_seed(T + K)
    q = torch.randn(B, T, H, 64, generator=g).bfloat16()
    k = torch.randn(B, S, H, 64, generator=g).bfloat16()
    v = torch.randn(B, S, H, 64, generator=g).bfloat16()
    pos = workloads.random_positions(B, T, S, K, seed=T + 1, invalid_fraction=inv)
    print(f"[dense attn_sum] B={B} T={T} S={S} H={H} K={K}", flush=True)
    o, attn, lse, _ = _run_attn(q, k, v, pos, scale=0.125)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos, 0.125)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(attn, ra, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)
    o2, lse2 = _run(q, k, v, pos, scale=0.125)
    assert torch.equal(o, o2) and torch.equal(lse, lse2), "attn_sum must not change o or lse"
    # every valid row's attention mass over the heads sums to H
    valid = ((pos >= 0) & (pos < S)).any(-1)
    torch.testing.assert_close(attn.sum(-1)[valid], torch.full((int(valid.sum()),), float(H)), atol=2e-3, rtol=1e-4)


def test_attn_sum_clustered_selections(gpu_device):
    # Rows selecting whole runs of consecutive keys (up to 32 selected keys of one query in a
    # 32-key sub-tile: eight rounds of the per-query score runs, with flushes of the score ring
    # between them), single keys, the last keys only with -1 padding, and random keys; every
    # row listed in a random order, so the list position j of a key is arbitrary. K = 100 (not
    # a multiple of 8), T and S ragged.
    B, T, S, H, K = 2, 300, 700, 4, 100
    g = torch.Generator().manual_seed(31)
    q = torch.randn(B, T, H, 64, generator=g).bfloat16()
    k = torch.randn(B, S, H, 64, generator=g).bfloat16()
    v = torch.randn(B, S, H, 64, generator=g).bfloat16()
    pos = torch.full((B, T, K), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(T):
            kind = t % 4
            if kind == 0:
                start = int(torch.randint(0, S - K, (1,), generator=g))
                row = torch.arange(start, start + K)
            elif kind == 1:
                starts = torch.randperm(S // 40, generator=g)[:3] * 40
                row = torch.cat([torch.arange(int(s0), int(s0) + 33) for s0 in starts] + [torch.tensor([S - 1])])
            elif kind == 2:
                row = torch.randperm(S, generator=g)[:K]
            else:
                row = torch.cat([torch.arange(S - 10, S), torch.full((K - 10,), -1)])
            pos[b, t] = row[torch.randperm(K, generator=g)].to(torch.int32)
    pos[1, 5] = -1                    # a row without any valid key
    pos[1, 6] = -1
    pos[1, 6, 17] = 3                 # a row with a single key
    print(f"[dense attn_sum] clustered B={B} T={T} S={S} H={H} K={K}", flush=True)
    o, attn, lse, _ = _run_attn(q, k, v, pos, scale=0.125)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos, 0.125)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(attn, ra, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)
    assert torch.all(attn[1, 5] == 0)
    torch.testing.assert_close(attn[1, 6, 17], torch.tensor(float(H)), atol=1e-5, rtol=1e-5)


def test_attn_sum_repeated_positions_and_bhtd(gpu_device):
    q, k, v = workloads.attention_inputs(1, 1, torch.bfloat16, tokens=200, seed=19)
    pos = workloads.random_positions(1, 200, 200, 13, seed=20)
    pos[0, 0, :] = -1
    pos[0, 70, :] = 7          # the gather kernel computes this block, attn_sum included
    o, attn, lse, _ = _run_attn(q, k, v, pos)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos)
    torch.testing.assert_close(o, ro, **TOL)
    torch.testing.assert_close(attn, ra, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(attn[0, 70], torch.full((13,), 16 / 13), atol=1e-5, rtol=1e-5)
    assert torch.all(attn[0, 0] == 0)
    o2, attn2, lse2, _ = _run_attn(q, k, v, pos, layout="bhtd")
    assert torch.equal(o, o2) and torch.equal(attn, attn2) and torch.equal(lse, lse2)


def test_fused_kl_rows_match_the_gather_kernel(gpu_device):
    B, T, H, K = 2, 700, 16, 256
    q, k, v = workloads.attention_inputs(1, B, torch.bfloat16, tokens=T, seed=23)
    pos = workloads.random_positions(B, T, T, K, seed=24, invalid_fraction=0.2)
    pos[1, 100, :4] = 5        # one flagged block: the gather kernel's fused KL
    z = torch.randn(B, T, K, generator=torch.Generator().manual_seed(25))
    od, ad, ld, kd = _run_attn(q, k, v, pos, kl=z)
    og, ag, lg, kg = _run_attn(q, k, v, pos, kl=z, path="gather")
    torch.testing.assert_close(ad, ag, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(kd, kg, atol=1e-5, rtol=1e-4)
    _, ad2, _, _ = _run_attn(q, k, v, pos)
    assert torch.equal(ad, ad2), "the fused KL must not change attn_sum"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_v_columns_outside_the_fp16_range(gpu_device, dtype):
    # V enters the product in fp16 scaled per (head, column) by 2^e: columns with |v| up to
    # 1e9 (bf16; 3e3 for fp16 inputs), down to 1e-9, and an all-zero column keep their
    # relative precision.
    B, T, S, H, K = 1, 200, 700, 2, 96
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, T, H, 64, generator=g).to(dtype)
    k = torch.randn(B, S, H, 64, generator=g).to(dtype)
    big = 1e9 if dtype == torch.bfloat16 else 3e3
    col = torch.ones(64)
    col[:16] = big
    col[16:32] = 1e-9 if dtype == torch.bfloat16 else 1e-4
    col[32] = 0.0
    v = (torch.randn(B, S, H, 64, generator=g) * col).to(dtype)
    pos = _distinct_positions(B, T, S, K, seed=5)
    print(f"[dense V scaling] {dtype}", flush=True)
    o, lse = _run(q, k, v, pos, scale=0.125)
    ro, rl = oatt.sparse_attention(q, k, v, pos, 0.125)[0::2]
    w = col.clamp_min(1e-30).view(1, 1, 1, 64)  # compare each column at its own scale
    torch.testing.assert_close(o / w, ro.float() / w, **TOL)
    assert torch.all(o[..., 32] == 0)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("H", [1, 3])
def test_odd_head_counts_and_scale(gpu_device, H):
    B, T, S, K = 2, 150, 333, 40
    g = torch.Generator().manual_seed(H)
    q = torch.randn(B, T, H, 64, generator=g).bfloat16()
    k = torch.randn(B, S, H, 64, generator=g).bfloat16()
    v = torch.randn(B, S, H, 64, generator=g).bfloat16()
    pos = _distinct_positions(B, T, S, K, seed=H + 3)
    print(f"[dense odd heads] H={H}", flush=True)
    o, lse = _run(q, k, v, pos, scale=0.3)
    ro, rl = oatt.sparse_attention(q, k, v, pos, 0.3)[0::2]
    torch.testing.assert_close(o, ro.float(), **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)


def _random_shape(seed):
    g = torch.Generator().manual_seed(1000 + seed)
    r = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    S = r(1, 2100)
    return dict(B=r(1, 2), T=r(1, 700), S=S, H=r(1, 5), K=r(1, min(S, 300)),
                inv=float(torch.rand(1, generator=g)) * 0.5,
                dtype=torch.bfloat16 if seed % 2 == 0 else torch.float16, seed=seed)


@pytest.mark.parametrize("case", [_random_shape(i) for i in range(12)],
                         ids=lambda c: f"B{c['B']}T{c['T']}S{c['S']}H{c['H']}K{c['K']}")
def test_random_shapes_against_the_oracle(gpu_device, case):
    # Seeded random sizes (T, S not multiples of 32 or 64, S below one tile, small K, ragged
    # -1 padding of distinct positions): o, lse and attn_sum at the stated bars.
    B, T, S, H, K, dt = case["B"], case["T"], case["S"], case["H"], case["K"], case["dtype"]
    g = torch.Generator().manual_seed(case["seed"])
    q = torch.randn(B, T, H, 64, generator=g).to(dt)
    k = torch.randn(B, S, H, 64, generator=g).to(dt)
    v = torch.randn(B, S, H, 64, generator=g).to(dt)
    pos = workloads.random_positions(B, T, S, K, seed=case["seed"], invalid_fraction=case["inv"])
    print(f"[dense random] {case}", flush=True)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos, 0.125)
    o, lse = _run(q, k, v, pos, scale=0.125)
    torch.testing.assert_close(o, ro.float(), **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)
    if K <= 1024:
        o2, attn, lse2, _ = _run_attn(q, k, v, pos, scale=0.125)
        torch.testing.assert_close(o2, ro.float(), **TOL)
        torch.testing.assert_close(attn, ra, atol=1e-4, rtol=1e-3)
        torch.testing.assert_close(lse2, rl, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("S", [63, 64, 65, 127, 128, 129, 191, 192, 193, 255, 256, 257, 383, 385])
def test_key_counts_around_the_128_key_tiles(gpu_device, S):
    # The plain pass sweeps keys in 128-key tiles (two 64-key halves; keys padded to 128), the
    # attn_sum pass in 64-key tiles: key counts just below, at and above each boundary, with
    # the last keys selected by every query, against the oracle.
    B, T, H = 1, 97, 2
    K = min(S, 48)
    g = torch.Generator().manual_seed(S)
    q = torch.randn(B, T, H, 64, generator=g).bfloat16()
    k = torch.randn(B, S, H, 64, generator=g).bfloat16()
    v = torch.randn(B, S, H, 64, generator=g).bfloat16()
    pos = _distinct_positions(B, T, S, K, seed=S + 1)
    # key S - 1 first in every row; an entry that already listed it becomes -1 (no repeats)
    rest = pos[..., 1:]
    pos[..., 1:] = torch.where(rest == S - 1, torch.full_like(rest, -1), rest)
    pos[..., 0] = S - 1
    print(f"[dense tiles] S={S}", flush=True)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos, 0.125)
    o, lse = _run(q, k, v, pos, scale=0.125)
    torch.testing.assert_close(o, ro.float(), **TOL)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-4)
    o2, attn, lse2, _ = _run_attn(q, k, v, pos, scale=0.125)
    torch.testing.assert_close(o2, ro.float(), **TOL)
    torch.testing.assert_close(attn, ra, atol=1e-4, rtol=1e-3)
    torch.testing.assert_close(lse2, rl, atol=1e-4, rtol=1e-4)


def _nonfinite_case(seed=41):
    # Batch 0: inf / nan in K and V rows that no query selects (the reference never reads
    # them). Batch 1: the same values in rows some queries do select.
    B, T, S, H, K = 2, 100, 1000, 4, 32
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).bfloat16()
    k = torch.randn(B, S, H, 64, generator=g).bfloat16()
    v = torch.randn(B, S, H, 64, generator=g).bfloat16()
    pos = _distinct_positions(B, T, S, K, seed=seed + 1)
    unused = [sorted(set(range(S)) - set(pos[b].reshape(-1).tolist())) for b in range(B)]
    assert len(unused[0]) >= 4, "the case needs keys that no query selects"
    k[0, unused[0][0], 1, 5] = float("inf")
    k[0, unused[0][1], 2, :] = float("nan")
    v[0, unused[0][2], 0, 9] = float("-inf")
    v[0, unused[0][3], 3, 0] = float("nan")
    used = pos[1, 17, 3].item(), pos[1, 70, 9].item()
    k[1, used[0], 1, 5] = float("inf")
    v[1, used[1], 2, 7] = float("nan")
    return q, k, v, pos


def _assert_same_nonfinite(got, want, tol):
    fin = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), fin), "non-finite entries differ from the oracle"
    torch.testing.assert_close(got[fin], want[fin], **tol)


@pytest.mark.parametrize("with_attn", [False, True])
def test_non_finite_k_v_take_the_gather_kernel(gpu_device, with_attn):
    # An inf or nan in a K or V row that no query selected must not reach any output (the
    # dense products would carry it through the -inf bias or the zero weight); the call
    # computes such a batch element with the gather kernel, as the reference reads only the
    # selected rows (sparse_index_flash_attn.py:205-216).
    q, k, v, pos = _nonfinite_case()
    print(f"[dense non-finite] with_attn={with_attn}", flush=True)
    ro, ra, rl = oatt.sparse_attention(q, k, v, pos)
    if with_attn:
        o, attn, lse, _ = _run_attn(q, k, v, pos, path="auto")
    else:
        o, lse = _run(q, k, v, pos, path="auto")
    assert torch.isfinite(o[0]).all() and torch.isfinite(lse[0]).all()
    torch.testing.assert_close(o[0], ro[0], **TOL)
    torch.testing.assert_close(lse[0], rl[0], atol=1e-4, rtol=1e-4)
    assert not torch.isfinite(ro[1]).all(), "batch 1 plants values in selected rows"
    _assert_same_nonfinite(o[1], ro[1], TOL)
    # the reference's softmax gives an lse of +inf where the online form gives nan
    nan = torch.tensor(float("nan"))
    _assert_same_nonfinite(torch.where(torch.isfinite(lse[1]), lse[1], nan),
                           torch.where(torch.isfinite(rl[1]), rl[1], nan), dict(atol=1e-4, rtol=1e-4))
    if with_attn:
        torch.testing.assert_close(attn[0], ra[0], atol=1e-4, rtol=1e-3)
        _assert_same_nonfinite(attn[1], ra[1], dict(atol=1e-4, rtol=1e-3))
    # finite inputs of the same shape still take the dense pass and agree with these rows
    k2, v2 = k.nan_to_num(nan=0.0, posinf=0.0, neginf=0.0), v.nan_to_num(nan=0.0, posinf=0.0, neginf=0.0)
    o2, lse2 = _run(q, k2, v2, pos, path="dense")
    torch.testing.assert_close(o2[0], o[0], **TOL)
