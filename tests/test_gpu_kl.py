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
