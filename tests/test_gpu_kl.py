"""GPU parity of the indexer KL training loss (gw_indexer_kl_fwd / gw_indexer_kl_bwd) against
the fp64 CPU oracle (oracle/kl_loss.py, the reference's explicit formulas from
easyvolcap/utils/custom_indexer/indexer_kl_fused.py:8-298).

Bar: the kernel computes in fp32 from inputs the oracle sees bit for bit (the same bf16 /
fp16 / fp32 values, upcast). Loss within 1e-5 relative; fp32 gradients within 1e-4
relative of the largest gradient magnitude in the row; 16-bit gradients within 2e-2 of it
(the path's 16-bit bar; one rounding of the output is 2^-9 relative in bf16).
"""
import pytest
import torch

from geoweave_amd.custom_indexer import sparse_indexer_kl_loss
from geoweave_amd.custom_indexer import indexer_kl_fused as klf
from oracle import kl_loss as okl

pytestmark = pytest.mark.gpu


def _inputs(B, T, K, dtype, seed, logits_dtype=None, zero_rows=0, sparse_frac=0.0):
    g = torch.Generator().manual_seed(seed)
    # attention mass: positive, heavy-tailed like softmax sums over heads
    a = torch.exp(torch.randn(B, T, K, generator=g) * 2.0)
    if sparse_frac:
        a = a * (torch.rand(B, T, K, generator=g) >= sparse_frac)
    if zero_rows:
        a.view(-1, K)[:zero_rows] = 0.0
    a = a / a.sum(-1, keepdim=True).clamp_min(1e-30)
    z = torch.randn(B, T, K, generator=g) * 3.0 + 1.5
    return a.to(dtype), z.to(logits_dtype or dtype)


def _term_scales(a, z, grad_out, eps):
    """Per-row magnitude of the terms each gradient is a difference of, for the tolerance:
    d_attn = (g - gbar) gs / (S + eps) and d_logits = (softmax(z) - p) gs cancel when the
    terms nearly agree (e.g. K = 1, where p = S / (S + eps)), and fp32 keeps ~1e-7 of the
    terms, not of the difference."""
    z = z.to(a.dtype).double().reshape(-1, z.shape[-1])  # logits are cast to attn's dtype
    a = a.double().reshape(-1, a.shape[-1])
    gs = float(grad_out) / a.shape[0]
    den = a.sum(-1, keepdim=True) + eps
    p = a / den
    lq = torch.log_softmax(z, -1)
    g = torch.log(p + eps) - lq + p / (p + eps)
    gbar = (p * g).sum(-1, keepdim=True)
    da_terms = torch.maximum(g.abs().amax(-1, keepdim=True), gbar.abs()) * gs / den
    dz_terms = torch.maximum(lq.exp(), p).amax(-1, keepdim=True) * gs
    return da_terms, dz_terms


def _check_grads(got, want, dtype, terms=None):
    got = got.double().cpu().reshape(want.shape[0] * want.shape[1], -1)
    want = want.reshape(got.shape)
    scale = want.abs().amax(-1, keepdim=True)
    if terms is not None:
        scale = torch.maximum(scale, 1e-2 * terms)  # fp32 cancellation floor (1e-6 of the terms)
    scale = scale.clamp_min(1e-30)
    rel = 1e-4 if dtype == torch.float32 else 2e-2
    err = (got - want).abs()
    bad = err > rel * scale
    assert not bool(bad.any()), f"max err/scale {float((err / scale).max()):.3e}"


def _run(a, z, eps, grad_out=1.0):
    ad = a.cuda().requires_grad_(True)
    zd = z.cuda().requires_grad_(True)
    loss = sparse_indexer_kl_loss(ad, zd, eps=eps)
    (loss * grad_out).backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), ad.grad.cpu(), zd.grad.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [1024, 37, 2048])
def test_kl_loss_matches_oracle(gpu_device, dtype, K):
    a, z = _inputs(2, 96, K, dtype, seed=100 + K)
    eps = 1e-6
    loss, da, dz = _run(a, z, eps, grad_out=3.0)
    want = okl.kl_loss(a, z, eps)
    assert loss.dtype == torch.float32 and loss.shape == ()
    assert abs(float(loss) - float(want)) <= 1e-5 * abs(float(want)) + 1e-7
    wda, wdz = okl.kl_loss_bwd(a, z, 3.0, eps)
    assert da.dtype == dtype and dz.dtype == dtype
    _check_grads(da, wda, dtype)
    _check_grads(dz, wdz, dtype)


def test_kl_loss_edges(gpu_device):
    # K = 1 (loss and d_logits vanish), K = 4096 (largest), zero-mass rows, sparse mass,
    # logits in another dtype than attn (cast to attn's dtype, indexer_kl_fused.py:171-172),
    # large eps.
    for (K, zero_rows, sparse, ldt, eps) in [(1, 0, 0.0, None, 1e-6), (4096, 3, 0.9, None, 1e-6),
                                             (512, 5, 0.99, torch.bfloat16, 1e-6), (300, 0, 0.5, None, 0.1)]:
        a, z = _inputs(1, 40, K, torch.float32, seed=K, logits_dtype=ldt, zero_rows=zero_rows, sparse_frac=sparse)
        print(f"[case] K={K} zero_rows={zero_rows} sparse={sparse} logits={ldt} eps={eps}", flush=True)
        loss, da, dz = _run(a, z, eps)
        want = okl.kl_loss(a, z, eps)
        assert abs(float(loss) - float(want)) <= 1e-5 * abs(float(want)) + 1e-7
        wda, wdz = okl.kl_loss_bwd(a, z, 1.0, eps)
        ta, tz = _term_scales(a, z, 1.0, eps)
        _check_grads(da, wda, torch.float32, ta)
        _check_grads(dz.float(), wdz, torch.float32 if ldt is None else ldt, tz)
        assert dz.dtype == (ldt or torch.float32)


def test_kl_row_losses_and_grad_out_on_device(gpu_device):
    # The backward reads dL/dloss from device memory: a grad_out tensor produced on the GPU
    # (no host value) must scale the gradients exactly as the reference's .item() does.
    a, z = _inputs(1, 64, 1024, torch.float32, seed=5)
    ad, zd = a.cuda(), z.cuda()
    rows = klf.kl_loss_forward(ad, zd, 1e-6).cpu()
    torch.testing.assert_close(rows.double(), okl.kl_row_losses(a, z, 1e-6), rtol=1e-5, atol=1e-7)
    go = torch.full((), 0.5, device="cuda") * 4.0
    da, dz = klf.kl_loss_backward(ad, zd, go, 1e-6)
    wda, wdz = okl.kl_loss_bwd(a, z, 2.0, 1e-6)
    _check_grads(da.cpu(), wda, torch.float32)
    _check_grads(dz.cpu(), wdz, torch.float32)


def test_kl_loss_is_bitwise_reproducible(gpu_device):
    a, z = _inputs(2, 500, 1024, torch.bfloat16, seed=9)
    r1 = _run(a, z, 1e-6)
    r2 = _run(a, z, 1e-6)
    for x, y in zip(r1, r2):
        assert torch.equal(x, y)


def test_kl_loss_at_layer_size_sampled_rows(gpu_device):
    # S = 32 views of 1374 tokens, K = 1024, the layer's bf16 p and top-k scores
    # (dsa_attention.py:5395-5411). Checked on 512 sampled rows, plus invariants on all.
    B, T, K = 1, 32 * 1374, 1024
    g = torch.Generator(device="cuda").manual_seed(77)
    a = torch.exp(torch.randn(B, T, K, device="cuda", generator=g) * 2.0)
    a = (a / a.sum(-1, keepdim=True)).to(torch.bfloat16)
    z = (torch.randn(B, T, K, device="cuda", generator=g) * 3.0).to(torch.bfloat16)
    rows = klf.kl_loss_forward(a, z, 1e-6)
    go = torch.ones((), device="cuda")
    da, dz = klf.kl_loss_backward(a, z, go, 1e-6)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(rows).all()) and float(rows.min()) > -1e-4  # KL >= 0 up to eps
    # d_logits sums to ~0 per row (softmax minus a distribution of mass S/(S+eps))
    assert float(dz.float().sum(-1).abs().max()) < 1e-2 / T
    sel = torch.randperm(T, generator=torch.Generator().manual_seed(3))[:512]
    ac, zc = a[0, sel.cuda()].cpu()[None], z[0, sel.cuda()].cpu()[None]
    torch.testing.assert_close(rows[sel.cuda()].cpu().double(), okl.kl_row_losses(ac, zc, 1e-6),
                               rtol=1e-5, atol=1e-6)
    wda, wdz = okl.kl_loss_bwd(ac, zc, 512.0 / T, 1e-6)  # gs = 1 / T for the sampled rows
    _check_grads(da[0, sel.cuda()].cpu()[None], wda, torch.bfloat16)
    _check_grads(dz[0, sel.cuda()].cpu()[None], wdz, torch.bfloat16)


# ------------------------------------------------- KL fused into the attention epilogue


def _attn_inputs(B, T, S, H, K, seed, invalid=True):
    from geoweave_amd import workloads

    q, k, v = workloads.attention_inputs(1, B, torch.bfloat16, tokens=max(T, S), heads=H, seed=seed)
    q, k, v = q[:, :T], k[:, :S], v[:, :S]
    g = torch.Generator().manual_seed(seed + 1)
    pos = torch.randint(0, S, (B, T, K), generator=g, dtype=torch.int32)
    if invalid:
        pos[0, 1, :] = -1            # a row with no valid key: attn_sum = 0, loss = 0
        pos[0, 2, ::3] = S           # out of range -> p = 0 for those entries
    z = (torch.randn(B, T, K, generator=g) * 2.0).bfloat16()
    return [x.contiguous().cuda() for x in (q, k, v, pos, z)]


@pytest.mark.parametrize("B,T,S,H,K", [(2, 300, 500, 16, 1024), (1, 257, 400, 16, 100), (1, 130, 300, 8, 1024),
                                       (1, 64, 2100, 16, 2048)])
def test_fused_kl_rows_match_standalone_and_oracle(gpu_device, B, T, S, H, K):
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import _flash_attn_forward

    q, k, v, pos, z = _attn_inputs(B, T, S, H, K, seed=K + H)
    rows = torch.empty(B * T, device=q.device, dtype=torch.float32)
    o, a, lse, _ = _flash_attn_forward(q, k, v, pos, softmax_scale=0.125, kl_logits=z, kl_eps=1e-6, kl_row_loss=rows)
    o2, a2, lse2, _ = _flash_attn_forward(q, k, v, pos, softmax_scale=0.125)
    want = klf.kl_loss_forward(a2, z.float().contiguous(), 1e-6)
    torch.cuda.synchronize()
    # the attention outputs are those of the unfused launch, bit for bit
    assert torch.equal(o, o2) and torch.equal(a, a2) and torch.equal(lse, lse2)
    torch.testing.assert_close(rows, want, rtol=1e-5, atol=1e-6)
    ref = okl.kl_row_losses(a2.cpu().double(), z.cpu().double(), 1e-6)
    torch.testing.assert_close(rows.cpu().double(), ref.reshape(-1), rtol=1e-5, atol=1e-6)
    assert float(rows[1]) == 0.0  # row (0, 1) has no valid key


def test_fused_kl_gradients_equal_the_two_calls(gpu_device):
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa

    q, k, v, pos, z = _attn_inputs(1, 400, 600, 16, 256, seed=5)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(6)).bfloat16().cuda()
    grads = []
    for fused in (True, False):
        qd, kd, vd, zd = (x.detach().clone().requires_grad_() for x in (q, k, v, z))
        if fused:
            o, attn, loss = klf.sparse_attention_kl_loss(qd, kd, vd, pos, zd, 1e-6, 0.125)
        else:
            o, attn = sifa.sparse_index_flash_attn_func(qd, kd, vd, pos, None, False, 0.125)
            loss = sparse_indexer_kl_loss(attn, zd, 1e-6)
        ((o.float() * do.float()).sum() + 3.0 * loss).backward()
        grads.append((float(loss.detach()), qd.grad, kd.grad, vd.grad, zd.grad))
    torch.cuda.synchronize()
    (l1, *g1), (l2, *g2) = grads
    assert abs(l1 - l2) <= 1e-5 * abs(l2) + 1e-7
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_fused_kl_detached_mass_equals_the_two_calls(gpu_device):
    # The reference presets' training (detach_input): the loss sees the attention mass
    # detached, so q, k, v get the gradient of o alone (the masked dense backward) and the
    # logits the KL gradient.
    from geoweave_amd.custom_flash_attn import _backward
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa

    from geoweave_amd import workloads

    q, k, v, _, z = _attn_inputs(1, 400, 600, 16, 256, seed=15, invalid=False)
    pos = workloads.distinct_positions(1, 400, 600, 256, seed=15).cuda()  # as top-k gives
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(16)).bfloat16().cuda()
    grads = []
    for fused in (True, False):
        qd, kd, vd, zd = (x.detach().clone().requires_grad_() for x in (q, k, v, z))
        if fused:
            o, attn, loss = klf.sparse_attention_kl_loss(qd, kd, vd, pos, zd, 1e-6, 0.125, detach_input=True)
        else:
            o, attn = sifa.sparse_index_flash_attn_func(qd, kd, vd, pos, None, False, 0.125)
            loss = sparse_indexer_kl_loss(attn.detach(), zd, 1e-6)
        ((o.float() * do.float()).sum() + 3.0 * loss).backward()
        assert _backward.last_path == "dense"
        grads.append((float(loss.detach()), qd.grad, kd.grad, vd.grad, zd.grad))
    torch.cuda.synchronize()
    (l1, *g1), (l2, *g2) = grads
    assert abs(l1 - l2) <= 1e-5 * abs(l2) + 1e-7
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_fused_kl_limits(gpu_device):
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import _flash_attn_forward

    q, k, v, pos, z = _attn_inputs(1, 8, 4000, 8, 1025, seed=9, invalid=False)
    rows = torch.empty(8, device=q.device, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="fused KL supports K <= 1024"):
        _flash_attn_forward(q, k, v, pos, softmax_scale=0.125, kl_logits=z, kl_row_loss=rows)
