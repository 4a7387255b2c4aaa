"""GPU checks of the aggregator host path around the sparse layer: dense/sparse block
equivalence when top-k covers every key, ``reuse_topk_groups`` (the reused layer skips its
indexer and attends over the source layer's keys), and HIP-graph replays against eager
runs (several replays with eager work between, each compared with its own eager result).

Small shapes: dim 256 (4 heads of 64, indexer 4 x 64), 4 + 4 blocks, a 2-block patch
embedding, 4 views of 70 x 70 images (5 x 5 patches + 5 special tokens = 30 tokens per
view, N = 120 global tokens).
"""
import pytest
import torch

from geoweave_amd import aggregator as agg
from geoweave_amd import dsa_layer

pytestmark = pytest.mark.gpu


def _model(indexer_layers="1-3", reuse=None, topk=32, seed=0):
    torch.manual_seed(seed)
    m = agg.Aggregator(dim=256, depth=4, num_heads=4, indexer_layers=indexer_layers, reuse_topk_groups=reuse,
                       topk=topk, patch_depth=2, img_size=70)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() >= 2:
                p.normal_(0.0, p.shape[-1] ** -0.5 if p.dim() == 2 else 0.02)
            elif name.endswith("gamma"):
                p.fill_(0.5)
            elif "norm" in name and name.endswith("weight"):
                p.normal_(1.0, 0.1)
            elif "w_proj" in name:
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02)
    return m.cuda().to(torch.bfloat16)


def _images(seed=1, S=4):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(1, S, 3, 70, 70, generator=g).cuda()


def test_sparse_blocks_equal_dense_blocks_when_topk_covers_all_keys(gpu_device):
    # With k = N every query attends to every key, so a sparse global block computes the
    # dense block's function; the two models share every weight but the indexer's.
    sparse = _model(indexer_layers="1-3", topk=120)
    dense = _model(indexer_layers="", topk=120)
    missing, unexpected = dense.load_state_dict(sparse.state_dict(), strict=False)
    assert not missing and all(".indexer." in k for k in unexpected)
    x = _images()
    out_s, start = sparse(x)
    out_d, _ = dense(x)
    torch.cuda.synchronize()
    assert start == 5 and len(out_s) == 4 and out_s[0].shape == (1, 4, 30, 512)
    for a, b in zip(out_s, out_d):
        torch.testing.assert_close(a.float(), b.float(), atol=3e-2, rtol=3e-2)


def test_reused_layers_skip_the_indexer_and_use_the_source_selection(gpu_device, monkeypatch):
    m = _model(indexer_layers="1-3", reuse="1:2-3", topk=32)
    calls = []
    real = dsa_layer.sparse_topk_indexer_inference_func

    def counting(*args, **kwargs):
        calls.append(args[0].shape)
        return real(*args, **kwargs)

    monkeypatch.setattr(dsa_layer, "sparse_topk_indexer_inference_func", counting)
    seen = {}
    for i in (1, 2, 3):
        attn = m.global_blocks[i].attn
        orig = attn.forward

        def spy(*a, _i=i, _orig=orig, **kw):
            out, idx = _orig(*a, **kw)
            seen[_i] = idx
            return out, idx

        monkeypatch.setattr(attn, "forward", spy)
    m(_images(seed=3))
    torch.cuda.synchronize()
    assert len(calls) == 1, "layers 2 and 3 must reuse layer 1's top-k"
    assert torch.equal(seen[2], seen[1]) and torch.equal(seen[3], seen[1])
    assert seen[1].shape == (1, 120, 32)


def test_graph_replays_match_eager(gpu_device):
    m = _model(indexer_layers="1-3", reuse="1:3", topk=32)
    graph = agg.AggregatorGraph(m)
    for rep in range(3):
        x = _images(seed=10 + rep)
        eager, _ = m(x)  # eager work between replays
        torch.cuda.synchronize()
        got, _ = graph(x)
        torch.cuda.synchronize()
        print(f"[replay] {rep}", flush=True)
        for a, b in zip(got, eager):
            torch.testing.assert_close(a.float(), b.float(), atol=1e-2, rtol=1e-2)


def test_source_downsample_option(gpu_device):
    # factor 2 over the 5 x 5 patch grid of each view: the sparse layers select through the
    # coarse selector (2 x 2 pooled cells + edge rows + specials); the rest of the model is
    # unchanged, and at factor 1 the option is off.
    exact = _model(indexer_layers="1-3", topk=32)
    coarse = _model(indexer_layers="1-3", topk=32)
    coarse.source_downsample_factor = 2
    x = _images(seed=4)
    out_e, _ = exact(x)
    out_c, _ = coarse(x)
    coarse.source_downsample_factor = 1
    out_off, _ = coarse(x)
    torch.cuda.synchronize()
    for a, b, c in zip(out_e, out_c, out_off):
        assert a.shape == b.shape and torch.isfinite(b.float()).all()
        assert torch.equal(a, c)
    assert any(not torch.equal(a, b) for a, b in zip(out_e[1:], out_c[1:]))
