"""GPU parity of the DSA layer glue (gw_dsa_glue_fwd) and of the sparse global-attention
layer built on it, against the fp32 CPU oracle (oracle/layer_glue.py, oracle/indexer.py,
oracle/attention.py).

Bar: the glue is fp32 math on the same 16-bit projection the oracle reads, rounded once
to bf16/fp16: within 2e-2 (abs + rel) of the oracle, the path's 16-bit bar. The layer is
checked stage by stage on the GPU's own intermediate tensors (as the C4 check feeds the
GPU indices to both sides): index sets tie-aware exact, the output within 2e-2.
"""
import pytest
import torch
import torch.nn.functional as F

from geoweave_amd import dsa_layer
from oracle import attention as oatt
from oracle import indexer as oidx
from oracle import layer_glue as olg
from oracle.topk_check import check_topk_rows

pytestmark = pytest.mark.gpu

TOL = dict(atol=2e-2, rtol=2e-2)


def _glue_case(B, N, H, Hi, dtype, seed, with_ln=True, with_rope=True, maxpos=38):
    g = torch.Generator().manual_seed(seed)
    lay = dsa_layer.GlueLayout(H, 64, Hi, 64)
    y = (torch.randn(B, N, lay.ldy, generator=g) * 2 + 0.5).to(dtype)
    norms = {}
    for key in ("q", "k", "idx_k"):
        norms[key] = (torch.rand(64, generator=g) + 0.5, torch.randn(64, generator=g) * 0.1) if with_ln else None
    pos = None
    if with_rope:
        pos = torch.randint(0, maxpos, (B, N, 2), generator=g)
        pos[:, :3] = 0  # special tokens sit at position (0, 0) (aggregator.py:521-526)
    return lay, y, norms, pos


def _run_glue(lay, y, norms, pos):
    dev = "cuda"
    nd = lambda key: (None, None) if norms[key] is None else tuple(t.to(dev) for t in norms[key])
    out = dsa_layer.dsa_glue_forward(y.to(dev), lay, nd("q"), nd("k"), nd("idx_k"), 1e-5,
                                     None if pos is None else pos.to(dev))
    torch.cuda.synchronize()
    return [t.float().cpu() for t in out]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_ln,with_rope", [(True, True), (False, True), (True, False), (False, False)])
def test_glue_matches_oracle(gpu_device, dtype, with_ln, with_rope):
    lay, y, norms, pos = _glue_case(2, 300, 16, 4, dtype, seed=5 + with_ln + 2 * with_rope,
                                    with_ln=with_ln, with_rope=with_rope)
    got = _run_glue(lay, y, norms, pos)
    want = olg.fused_projection_glue(None, None, None, dict(H=16, D=64, Hi=4, Di=64), norms, pos,
                                     y=y[..., :lay.width].float())
    for name, a, b in zip(("q", "k", "v", "idx_q", "idx_k", "idx_w"), got, want):
        torch.testing.assert_close(a, b, **TOL, msg=lambda m: f"{name}: {m}")


def test_glue_at_layer_size_sampled_rows(gpu_device):
    # S = 32 views of 1374 tokens, the layer's bf16 projection; oracle on sampled rows.
    lay, y, norms, pos = _glue_case(1, 32 * 1374, 16, 4, torch.bfloat16, seed=32)
    got = _run_glue(lay, y, norms, pos)
    rows = torch.randperm(y.shape[1], generator=torch.Generator().manual_seed(1))[:2048]
    want = olg.fused_projection_glue(None, None, None, dict(H=16, D=64, Hi=4, Di=64), norms, pos[:, rows],
                                     y=y[:, rows, :lay.width].float())
    for a, b in zip(got, want):
        torch.testing.assert_close(a[:, rows], b, **TOL)


def test_glue_rejects_bad_layouts(gpu_device):
    lay = dsa_layer.GlueLayout(16, 64, 4, 64)
    y = torch.zeros(1, 8, lay.ldy - 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        dsa_layer.dsa_glue_forward(y, lay)


def _layer(dim=1024, seed=0):
    torch.manual_seed(seed)
    m = dsa_layer.SparseGlobalAttention(dim=dim, num_heads=dim // 64, topk=256)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * (0.03 if p.dim() > 1 else 0.5))
        m.q_norm.weight.add_(1.0)
        m.k_norm.weight.add_(1.0)
        m.indexer.k_norm.weight.add_(1.0)
        m.indexer.w_proj.bias.fill_(1.0)
    return m


def test_sparse_global_attention_layer_stage_by_stage(gpu_device):
    B, N, dim = 1, 1500, 1024
    m = _layer(dim).cuda()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, N, dim, generator=g).bfloat16()
    pos = torch.randint(0, 38, (B, N, 2), generator=g)
    out, idx = m(x.cuda(), pos.cuda(), return_topk=True)
    torch.cuda.synchronize()

    # 1) projection + glue on the GPU vs the oracle on the same bf16 projection y
    w, b = m.fused_projection(torch.bfloat16)
    y = F.linear(x.cuda(), w, b)
    lay = m.layout
    norms = {"q": (m.q_norm.weight.detach().float().cpu(), m.q_norm.bias.detach().float().cpu()),
             "k": (m.k_norm.weight.detach().float().cpu(), m.k_norm.bias.detach().float().cpu()),
             "idx_k": (m.indexer.k_norm.weight.detach().float().cpu(), m.indexer.k_norm.bias.detach().float().cpu())}
    gq, gk, gv, giq, gik, giw = dsa_layer.dsa_glue_forward(
        y, lay, *[tuple(t.cuda() for t in norms[key]) for key in ("q", "k", "idx_k")], 1e-5, pos.cuda())
    want = olg.fused_projection_glue(None, None, None, dict(H=16, D=64, Hi=4, Di=64), norms, pos,
                                     y=y[..., :lay.width].float().cpu())
    for a, bb in zip((gq, gk, gv, giq, gik, giw), want):
        torch.testing.assert_close(a.float().cpu(), bb, **TOL)

    # 2) the layer's indices: exact top-256 of the oracle scores over the GPU's indexer q/k/w
    ref_scores = oidx.indexer_scores(giq.cpu(), gik.cpu(), giw.cpu(), None, 0.125)[0]
    rep = check_topk_rows(ref_scores, idx[0].cpu(), 256)
    assert rep.ok, rep

    # 3) attention over those indices, then the output projection, in fp32 on the CPU
    o, _, _ = oatt.sparse_attention(gq.cpu(), gk.cpu(), gv.cpu(), idx.cpu(), 0.125)
    ref = F.linear(o.to(torch.bfloat16).float().reshape(B, N, dim), m.proj.weight.detach().bfloat16().float().cpu(),
                   m.proj.bias.detach().bfloat16().float().cpu())
    torch.testing.assert_close(out.float().cpu(), ref, **TOL)


def test_score_dtype_float16_layer_at_s4(gpu_device, monkeypatch):
    # The reference preset's precision mode (geoweave/configs/vggt.json:35, "score_dtype":
    # "float16" under bf16 activations; dsa_attention.py:4943-4948, :617-620): after the glue
    # the attention q/k/v and the indexer q/k/w are cast to fp16, top-k and attention run in
    # fp16, and the output returns to bf16 before proj. C1's shape: S = 4 views of 1374
    # tokens, 16 heads of 64, top-k 1024.
    B, N, dim, K = 1, 4 * 1374, 1024, 1024
    m = _layer(dim, seed=11)
    m.topk = K
    m.score_dtype = dsa_layer.parse_score_dtype("float16")
    m = m.cuda()
    seen = []
    real = dsa_layer.sparse_index_flash_attn_inference_func

    def spy(q, k, v, idx, **kw):
        seen.append((q.dtype, k.dtype, v.dtype))
        return real(q, k, v, idx, **kw)

    monkeypatch.setattr(dsa_layer, "sparse_index_flash_attn_inference_func", spy)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(B, N, dim, generator=g).bfloat16()
    pos = torch.randint(0, 38, (B, N, 2), generator=g)
    out, idx = m(x.cuda(), pos.cuda(), return_topk=True)
    torch.cuda.synchronize()
    assert seen == [(torch.float16,) * 3]
    assert out.dtype == torch.bfloat16

    w, b = m.fused_projection(torch.bfloat16)
    y = F.linear(x.cuda(), w, b)
    norms = [(t.weight.detach().cuda(), t.bias.detach().cuda()) for t in (m.q_norm, m.k_norm, m.indexer.k_norm)]
    glue = dsa_layer.dsa_glue_forward(y, m.layout, *norms, 1e-5, pos.cuda())
    gq, gk, gv, giq, gik, giw = [t.to(torch.float16).cpu() for t in glue]
    # indices: exact top-1024 of the oracle scores over the fp16 indexer q/k/w
    ref_scores = oidx.indexer_scores(giq, gik, giw, None, 0.125)[0]
    rep = check_topk_rows(ref_scores, idx[0].cpu(), K)
    assert rep.ok, rep
    # attention over those indices on the fp16 q/k/v, o rounded to fp16 then bf16, proj
    o, _, _ = oatt.sparse_attention(gq, gk, gv, idx.cpu(), 0.125)
    o = o.to(torch.float16).to(torch.bfloat16).float()
    ref = F.linear(o.reshape(B, N, dim), m.proj.weight.detach().bfloat16().float().cpu(),
                   m.proj.bias.detach().bfloat16().float().cpu())
    torch.testing.assert_close(out.float().cpu(), ref, **TOL)


def test_pi3_global_attention_layer(gpu_device):
    # Pi3's DSA decoder attention (block.py:345-447 via pi3_training.py:245-275): qkv bias,
    # q/k LayerNorm, Pi3's RoPE2D (pos_embed.py:112-160) at base 100 over Pi3's positions
    # (5 register tokens at (0, 0), the 37 x 37 grid + 1), fp16 scores; 2 views in one
    # global layer. Stage by stage against the oracle with Pi3's rotation.
    S, P, dim, K = 2, 1374, 1024, 1024
    torch.manual_seed(31)
    m = dsa_layer.pi3_global_attention(dim=dim, topk=K)
    with torch.no_grad():
        for prm in m.parameters():
            prm.copy_(torch.randn_like(prm) * (0.03 if prm.dim() > 1 else 0.5))
        for norm in (m.q_norm, m.k_norm, m.indexer.k_norm):
            norm.weight.add_(1.0)
        m.indexer.w_proj.bias.fill_(1.0)
    m = m.cuda()
    g = torch.Generator().manual_seed(32)
    x = torch.randn(1, S * P, dim, generator=g).bfloat16()
    pos = dsa_layer.grid_positions(S, 37, 37).reshape(1, S * P, 2)
    assert torch.equal(pos.long(), olg.pi3_positions(S, 37, 37).reshape(1, S * P, 2))
    out, idx = m(x.cuda(), pos.cuda(), return_topk=True)
    torch.cuda.synchronize()

    w, b = m.fused_projection(torch.bfloat16)
    y = F.linear(x.cuda(), w, b)
    norms = {"q": (m.q_norm.weight.detach().float().cpu(), m.q_norm.bias.detach().float().cpu()),
             "k": (m.k_norm.weight.detach().float().cpu(), m.k_norm.bias.detach().float().cpu()),
             "idx_k": (m.indexer.k_norm.weight.detach().float().cpu(), m.indexer.k_norm.bias.detach().float().cpu())}
    glue = dsa_layer.dsa_glue_forward(y, m.layout, *[tuple(t.cuda() for t in norms[key]) for key in ("q", "k", "idx_k")],
                                      1e-5, pos.cuda())
    want = olg.fused_projection_glue(None, None, None, dict(H=16, D=64, Hi=4, Di=64), norms, pos.long(),
                                     y=y[..., :m.layout.width].float().cpu(), rope=olg.rope2d_pi3)
    for a, bb in zip(glue, want):
        torch.testing.assert_close(a.float().cpu(), bb, **TOL)
    gq, gk, gv, giq, gik, giw = [t.to(torch.float16).cpu() for t in glue]
    ref_scores = oidx.indexer_scores(giq, gik, giw, None, 0.125)[0]
    rep = check_topk_rows(ref_scores, idx[0].cpu(), K)
    assert rep.ok, rep
    o, _, _ = oatt.sparse_attention(gq, gk, gv, idx.cpu(), 0.125)
    o = o.to(torch.float16).to(torch.bfloat16).float()
    ref = F.linear(o.reshape(1, S * P, dim), m.proj.weight.detach().bfloat16().float().cpu(),
                   m.proj.bias.detach().bfloat16().float().cpu())
    torch.testing.assert_close(out.float().cpu(), ref, **TOL)


def test_query_chunked_stream_equals_the_whole_layer(gpu_device):
    # The query-chunked sparse stream (dsa_attention.py:1017-1283) selects and attends per
    # chunk of queries; rows are independent, so the output equals the unchunked layer's
    # (up to the summation order of equal index sets).
    B, N, dim = 1, 2500, 1024
    m = _layer(dim).cuda()
    g = torch.Generator().manual_seed(8)
    x = torch.randn(B, N, dim, generator=g).bfloat16().cuda()
    pos = torch.randint(0, 38, (B, N, 2), generator=g).cuda()
    whole = m(x, pos)
    chunked = m(x, pos, query_chunk=700)  # ragged last chunk
    torch.cuda.synchronize()
    torch.testing.assert_close(chunked.float(), whole.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("with_ln,with_rope", [(True, True), (False, True), (True, False)])
def test_glue_backward_matches_autograd_of_the_oracle(gpu_device, with_ln, with_rope):
    lay, y, norms, pos = _glue_case(2, 257, 16, 4, torch.bfloat16, seed=40 + with_ln + 2 * with_rope,
                                    with_ln=with_ln, with_rope=with_rope)
    g = torch.Generator().manual_seed(41)
    gq, gk = (torch.randn(2, 257, 16, 64, generator=g).bfloat16() for _ in range(2))
    giq, gik = (torch.randn(2, 257, 4, 64, generator=g).bfloat16() for _ in range(2))
    giw = torch.randn(2, 257, 4, generator=g).bfloat16()
    dev = "cuda"
    yd = y.to(dev).requires_grad_()
    nd = {k: None if v is None else tuple(t.to(dev).requires_grad_() for t in v) for k, v in norms.items()}
    pos32 = cos = sin = None
    n_rope = 0
    if pos is not None:
        pos32 = pos.to(dev, torch.int32)
        n_rope = int(pos.max()) + 1
        cos, sin = dsa_layer.rope2d_tables(n_rope, 100.0, dev)
    flat = lambda key: (None, None) if nd[key] is None else nd[key]
    outs = dsa_layer.GlueFunction.apply(yd, *flat("q"), *flat("k"), *flat("idx_k"), lay, 1e-5, pos32, cos, sin,
                                        n_rope)
    torch.autograd.backward(outs, [t.to(dev) for t in (gq, gk, giq, gik, giw)])
    torch.cuda.synchronize()

    yr = y[..., :lay.width].float().requires_grad_()
    nr = {k: None if v is None else tuple(t.clone().requires_grad_() for t in v) for k, v in norms.items()}
    q, k, v, iq, ik, iw = olg.fused_projection_glue(None, None, None, dict(H=16, D=64, Hi=4, Di=64), nr, pos, y=yr)
    loss = sum((a * b.float()).sum() for a, b in zip((q, k, iq, ik, iw), (gq, gk, giq, gik, giw)))
    loss.backward()
    got = yd.grad.float().cpu()
    torch.testing.assert_close(got[..., :lay.width], yr.grad, **TOL)
    assert float(got[..., lay.v_off:lay.v_off + 16 * 64].abs().max()) == 0.0  # v block left to the v view
    assert float(got[..., lay.width:].abs().max()) == 0.0
    if with_ln:
        for key in ("q", "k", "idx_k"):
            for a, b in zip(nd[key], nr[key]):
                err = float((a.grad.cpu() - b.grad).norm() / b.grad.norm())
                assert err < 2e-3, (key, err)


@pytest.mark.parametrize("score_dtype", [None, "float16", "float32"])
def test_layer_training_gradients_match_the_fp32_pipeline(gpu_device, score_dtype):
    # forward_train + KL loss through every HIP backward (glue, indexer, attention, KL) vs
    # autograd of the fp32 CPU pipeline on the same bf16 inputs/weights and the GPU's own
    # top-k indices. Bar: per-tensor relative error (norm) within 2e-2. With score_dtype
    # "float16" the indexer and attention run on fp16 casts of the glue's bf16 outputs and
    # their gradients return through the casts; with "float32" the indexer runs in fp32 and
    # the attention in bf16.
    from geoweave_amd.custom_indexer import sparse_indexer_kl_loss
    from oracle import kl_loss as okl

    B, N, dim, K = 1, 600, 256, 64
    torch.manual_seed(3)
    m = dsa_layer.SparseGlobalAttention(dim=dim, num_heads=4, topk=K, score_dtype=score_dtype)
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.copy_(torch.randn_like(p) * (dim ** -0.5 if p.dim() == 2 else 0.1))
        for norm in (m.q_norm, m.k_norm, m.indexer.k_norm):
            norm.weight.add_(1.0)
        m.indexer.w_proj.bias.fill_(1.0)
    m = m.to(torch.bfloat16)
    ref_m = {n: p.detach().float().clone().requires_grad_() for n, p in m.named_parameters()}
    m = m.cuda()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, N, dim, generator=g).bfloat16()
    pos = torch.randint(0, 12, (B, N, 2), generator=g)
    G = torch.randn(B, N, dim, generator=g) * 0.1

    xd = x.cuda().requires_grad_()
    out, attn, scores, idx = m.forward_train(xd, pos.cuda())
    assert scores.dtype == {None: torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[score_dtype]
    assert out.dtype == torch.bfloat16
    p = attn.to(torch.bfloat16)
    p = p / (p.sum(-1, keepdim=True) + 1e-6)
    loss = (out.float() * G.cuda()).sum() + sparse_indexer_kl_loss(p, scores, 1e-6)
    loss.backward()
    torch.cuda.synchronize()

    # fp32 reference pipeline with the GPU's indices
    xr = x.float().requires_grad_()
    W = torch.cat([ref_m[f"{n}.weight"] for n in ("qkv", "indexer.q_proj", "indexer.k_proj", "indexer.w_proj")])
    bvec = torch.cat([ref_m[f"{n}.bias"] for n in ("qkv", "indexer.q_proj", "indexer.k_proj", "indexer.w_proj")])
    norms = {"q": (ref_m["q_norm.weight"], ref_m["q_norm.bias"]), "k": (ref_m["k_norm.weight"], ref_m["k_norm.bias"]),
             "idx_k": (ref_m["indexer.k_norm.weight"], ref_m["indexer.k_norm.bias"])}
    q, k, v, iq, ik, iw = olg.fused_projection_glue(xr, W, bvec, dict(H=4, D=64, Hi=4, Di=64), norms, pos)
    idx_c = idx.cpu()
    sc = oidx.selected_scores(iq, ik, iw, idx_c, 0.125)
    o, attn_r = oatt.sparse_attention_differentiable(q, k, v, idx_c, 0.125)
    outr = torch.nn.functional.linear(o.reshape(B, N, dim), ref_m["proj.weight"], ref_m["proj.bias"])
    pr = attn_r / (attn_r.sum(-1, keepdim=True) + 1e-6)
    lossr = (outr * G).sum() + okl.kl_loss_autograd(pr, sc, 1e-6)
    lossr.backward()

    def rel(a, b):
        return float((a.float().cpu() - b).norm() / b.norm())

    assert rel(out.detach(), outr.detach()) < 2e-2
    assert rel(xd.grad, xr.grad) < 2e-2
    params = dict(m.named_parameters())
    for name in ("qkv.weight", "qkv.bias", "q_norm.weight", "k_norm.bias", "proj.weight",
                 "indexer.q_proj.weight", "indexer.k_proj.weight", "indexer.k_norm.weight", "indexer.w_proj.weight"):
        assert params[name].grad is not None, name
        assert rel(params[name].grad, ref_m[name].grad) < 2e-2, (name, rel(params[name].grad, ref_m[name].grad))
