#!/usr/bin/env python3
"""Benchmark of the sparse global-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--views 32] [--no-cpu-baseline]

One step = one pass of the hot path over one layer of synthetic input, with every input
already resident in HBM: the fused lightning-indexer score + exact top-k
(``sparse_topk_indexer_inference_func``), then the sparse-index attention forward over the
selected positions (``sparse_index_flash_attn_inference_func``, no ``attn_sum``). This is
the inference path of one VGGT/Pi3 global-attention layer. The workload is BASELINE
config "Metric row": B = 1, S = 32 views x 1374 tokens (N = 43,968), 16 heads x 64,
indexer 4 heads x 64, top-k 1024, bf16.

Printed: ONE JSON line. ``value`` = indexer ms + attention-forward ms per layer (lower is
better). ``roofline`` = the attention forward (the dominant call) against the roofline of
what it executes, timed live with HIP events on the stream the kernels run on: for the
masked dense pass the bf16 MFMA roofline on its flops (every (query, key) product,
4*B*T*S*H*D), for the gather kernel the HBM roofline on the gathered K/V bytes.
``attn_effective_gathered_bandwidth`` = the sparse formulation's gathered bytes over the
same time (a rate, not a roofline, for the dense pass). ``roofline_indexer`` = the indexer
against the bf16 MFMA roofline. ``cpu_baseline`` = the fp32 CPU oracle (the restatement of
the reference's torch backend) on a fixed sample of query rows of the same layer (median of
3 passes, scaled to the full layer), plus config C1 timed in full (median of 3 runs) beside
the GPU's C1 time.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "sparse global-attn layer fwd ms + indexer top-k ms at S=32 views, k=1024 (1 GPU)"


def attn_fwd_algorithmic_bytes(B, T, H, D, K, elt=2):
    """Gathered K and V rows (K per query, shared by the H heads) + q read + o write +
    int32 positions: B*T*K*H*D*2*elt + 2*B*T*H*D*elt + 4*B*T*K."""
    return B * T * K * H * D * 2 * elt + 2 * B * T * H * D * elt + 4 * B * T * K


def attn_fwd_dense_flops(B, T, S, H, D):
    """4 * B * T * S * H * D: the Q.K^T and P.V products over every (query, key) pair of the
    masked dense formulation (what the kernel executes: one MFMA flop per counted flop)."""
    return 4 * B * T * S * H * D


def indexer_algorithmic_flops(B, T, S, Hi, Di):
    """2 * B * T * S * Hi * Di (the q k^T products over all indexer heads)."""
    return 2 * B * T * S * Hi * Di


def read_traffic_summary(path: Path):
    """HBM bytes per launch of the attention forward, from the committed rocprofv3 PMC
    summary (a line ``traffic_bytes_per_launch: <int>``), or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def train_step_c4(steps: int = 5, warmup: int = 2, views: int = 24, batch: int = 2, topk: int = 1024):
    """Config C4: one training step of the layer's hot path through autograd, B=2, S=24
    views (N=32,976), bf16: indexer top-k forward, sparse attention forward with
    attn_sum, the indexer KL loss on the layer's normalised attention mass
    (dsa_attention.py:5395-5411: attn cast to q's dtype, p = attn / (sum + eps),
    sparse_indexer_kl_loss(p, topk_scores)), and the backward of o (a random dO) and of
    the KL loss. As in the reference presets (detach_input, vggt.json:17,
    dsa_attention.py:4694-4695) the loss sees the attention mass detached: it trains the
    indexer (KL backward, the indexer's masked dense backward) and the attention gets the
    gradient of o alone (the masked dense backward): no CSR is built. ``kl_into_attention`` times the same step with
    the mass not detached (the KL gradient also flows into q, k, v: the CSR backward with
    dattn). Times each phase with HIP events on the launch stream."""
    import torch

    from geoweave_amd import _csr, workloads
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import sparse_index_flash_attn_func
    from geoweave_amd.custom_indexer import sparse_indexer_kl_loss, sparse_topk_indexer_func
    from geoweave_amd.custom_indexer.indexer_kl_fused import sparse_attention_kl_loss

    dev = torch.device("cuda", 0)
    lay = workloads.layer_inputs(views, batch, torch.bfloat16)
    qi, ki, wi, q, k, v = (x.to(dev).requires_grad_() for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v))
    g = torch.Generator().manual_seed(views)
    B, T, H, D = q.shape
    do = torch.randn(B, T, H, D, generator=g).bfloat16().to(dev)
    stream = torch.cuda.current_stream(dev)
    eps = 1e-6

    def one(ev=None, fused=False, detach=True):
        for x in (qi, ki, wi, q, k, v):
            x.grad = None
        _csr.clear_cache()
        if ev:
            ev[0].record(stream)
        idx, sc = sparse_topk_indexer_func(qi, ki, wi, None, topk, 0.125, 256, 0)
        if fused:
            # KL on the attention mass computed in the attention epilogue (one launch)
            o, attn, kl = sparse_attention_kl_loss(q, k, v, idx, sc, eps, 0.125, detach_input=detach)
            if ev:
                ev[1].record(stream)
                ev[2].record(stream)
        else:
            o, attn = sparse_index_flash_attn_func(q, k, v, idx, None, False, 0.125)
            if ev:
                ev[1].record(stream)
            p = (attn.detach() if detach else attn).to(q.dtype)
            p = p / (p.sum(dim=-1, keepdim=True) + eps)
            kl = sparse_indexer_kl_loss(p, sc, eps)
            if ev:
                ev[2].record(stream)
        torch.autograd.backward([o, kl], [do, None])
        if ev:
            ev[3].record(stream)

    def timed(fused, detach=True):
        for _ in range(warmup):
            one(fused=fused, detach=detach)
        torch.cuda.synchronize()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
        for i in range(steps):
            one(evs[i], fused, detach)
        torch.cuda.synchronize()
        return [statistics.mean(e[j].elapsed_time(e[j + 1]) for e in evs) for j in range(3)]

    fwd, kl_ms, bwd = timed(False)
    f_fwd, _, f_bwd = timed(True)
    n_fwd, n_kl, n_bwd = timed(False, detach=False)
    gather = batch * T * topk * H * D * 2 * 2
    return {
        "workload": f"C4 training step: B={batch}, S={views} views (N={T}), H={H}, D={D}, top-k {topk}, bf16, "
                    "indexer + attention forward (attn_sum on), indexer KL loss on the detached attention mass "
                    "(the reference presets' detach_input), backward through autograd",
        "fwd_ms": round(fwd, 3),
        "kl_loss_fwd_ms": round(kl_ms, 3),
        "bwd_ms": round(bwd, 3),
        "step_ms": round(fwd + kl_ms + bwd, 3),
        "fused_kl": {
            "note": "indexer KL on the fp32 attention mass computed in the attention epilogue "
                    "(sparse_attention_kl_loss) instead of a separate loss kernel on the bf16-normalised mass",
            "fwd_ms": round(f_fwd, 3),
            "bwd_ms": round(f_bwd, 3),
            "step_ms": round(f_fwd + f_bwd, 3),
        },
        "kl_into_attention": {
            "note": "same step with the attention mass not detached: the KL gradient also flows into q, k, v "
                    "(attention backward with dattn: the CSR path)",
            "fwd_ms": round(n_fwd, 3),
            "kl_loss_fwd_ms": round(n_kl, 3),
            "bwd_ms": round(n_bwd, 3),
            "step_ms": round(n_fwd + n_kl + n_bwd, 3),
        },
        "attn_gathered_bytes_fwd": gather,
        "attn_gathered_bytes_bwd": 2 * gather,
        "attn_dense_bwd_flops": 10 * batch * T * T * H * D,
    }


def long_context_c3(steps: int = 5, warmup: int = 2, views: int = 64, topk: int = 1024):
    """Config C3: the inference step (indexer top-k + sparse attention forward) at S=64
    views (N=87,936), B=1, bf16; HIP-event timing per phase on the launch stream."""
    import torch

    from geoweave_amd import workloads
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import (
        sparse_index_flash_attn_inference_func,
    )
    from geoweave_amd.custom_indexer import sparse_topk_indexer_inference_func

    dev = torch.device("cuda", 0)
    lay = workloads.layer_inputs(views, 1, torch.bfloat16)
    qi, ki, wi, q, k, v = (x.to(dev) for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v))
    del lay
    stream = torch.cuda.current_stream(dev)
    empty_mask = qi.new_empty(0)

    def one(ev=None):
        if ev:
            ev[0].record(stream)
        idx, _ = sparse_topk_indexer_inference_func(qi, ki, wi, empty_mask, topk, 0.125, 256, 0)
        if ev:
            ev[1].record(stream)
        sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=0.125)
        if ev:
            ev[2].record(stream)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        one(evs[i])
    torch.cuda.synchronize()
    idx_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    att_ms = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)
    B, T, H, D = q.shape
    att_bytes = attn_fwd_algorithmic_bytes(B, T, H, D, topk)
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa

    attn_path = "dense" if sifa._use_dense(T, topk, H, D, 0.125) else "gather"

    # The query-chunked stream (dsa_attention.py:1017-1283): same work, the indices and the
    # indexer workspace live per chunk of 16384 queries. Peak memory above the inputs.
    from geoweave_amd.dsa_layer import sparse_attention_streaming

    def peak_of(fn):
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated(dev)
        torch.cuda.reset_peak_memory_stats(dev)
        fn()
        torch.cuda.synchronize()
        return (torch.cuda.max_memory_allocated(dev) - base) / 1e9

    chunk = 16384
    stream = lambda: sparse_attention_streaming(q, k, v, qi, ki, wi, topk, chunk, 0.125, 0.125)
    stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream(dev))
    for _ in range(steps):
        stream()
    e1.record(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    stream_ms = e0.elapsed_time(e1) / steps
    peak_whole = peak_of(lambda: one())
    peak_stream = peak_of(stream)
    return {
        "stream_query_chunk": chunk,
        "stream_ms": round(stream_ms, 3),
        "peak_extra_gb_whole": round(peak_whole, 2),
        "peak_extra_gb_stream": round(peak_stream, 2),
        "workload": f"C3 long context: B=1, S={views} views (N={T}), H={H}, D={D}, top-k {topk}, bf16, "
                    "indexer + sparse attention forward",
        "value_ms": round(idx_ms + att_ms, 3),
        "indexer_ms": round(idx_ms, 3),
        "attn_fwd_ms": round(att_ms, 3),
        "attn_path": attn_path,
        "attn_fwd_gbs": round(att_bytes / (att_ms * 1e-3) / 1e9, 1),
        "indexer_tflops": round(indexer_algorithmic_flops(B, T, T, qi.shape[2], qi.shape[3]) / (idx_ms * 1e-3) / 1e12, 2),
    }


def layer_forward_s32(steps: int = 5, warmup: int = 2, views: int = 32, topk: int = 1024):
    """The whole sparse global-attention layer forward at S=32 views (N=43,968), B=1, bf16,
    random-init weights: fused projection GEMM (hipBLASLt via torch), layer glue
    (gw_dsa_glue_fwd), indexer top-k, sparse attention, output projection. HIP events per
    phase on the launch stream. Also times the same glue written as separate torch ops
    (LayerNorm, rotary gathers and concatenations, casts: the reference's unfused order,
    dsa_attention.py:4928-4948 and indexer.py:302-328) for the fusion comparison."""
    import torch
    import torch.nn.functional as F

    from geoweave_amd import dsa_layer, workloads
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import (
        sparse_index_flash_attn_inference_func,
    )
    from geoweave_amd.custom_indexer import sparse_topk_indexer_inference_func

    dev = torch.device("cuda", 0)
    m = workloads.init_layer_(dsa_layer.SparseGlobalAttention(topk=topk)).to(dev)
    x, pos = workloads.layer_module_inputs(views)
    x, pos = x.to(dev), pos.to(dev)
    B, N, dim = x.shape
    lay = m.layout
    w, b = m.fused_projection(torch.bfloat16)
    pw = m.proj.weight.detach().to(torch.bfloat16)
    pb = m.proj.bias.detach().to(torch.bfloat16)
    norms = [dsa_layer._ln_params(n) for n in (m.q_norm, m.k_norm, m.indexer.k_norm)]
    n_rope = int(pos.max()) + 1
    cos, sin = dsa_layer.rope2d_tables(n_rope, 100.0, dev)
    empty = x.new_empty(0)
    stream = torch.cuda.current_stream(dev)

    def one(ev=None):
        rec = (lambda i: ev[i].record(stream)) if ev else (lambda i: None)
        rec(0)
        y = F.linear(x, w, b)
        rec(1)
        q, k, v, iq, ik, iw = dsa_layer.dsa_glue_forward(y, lay, *norms, 1e-5, pos, 100.0, n_rope)
        rec(2)
        idx, _ = sparse_topk_indexer_inference_func(iq, ik, iw, empty, topk, 0.125, 256, 0)
        rec(3)
        o, _ = sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=0.125)
        rec(4)
        F.linear(o.reshape(B, N, dim), pw, pb)
        rec(5)

    def rope_torch(t, p):  # t [B, N, h, 64] -> rotary as rope.py:133-200 in torch ops
        t = t.permute(0, 2, 1, 3)
        out = []
        for half, pp in ((t[..., :32], p[..., 0]), (t[..., 32:], p[..., 1])):
            c = torch.cat((cos, cos), -1)[pp.long()][:, None]
            s_ = torch.cat((sin, sin), -1)[pp.long()][:, None]
            out.append(half * c + torch.cat((-half[..., 16:], half[..., :16]), -1) * s_)
        return torch.cat(out, -1).permute(0, 2, 1, 3)

    def torch_glue(y):
        H, Hi = lay.H, lay.Hi
        q = y[..., lay.q_off:lay.q_off + H * 64].reshape(B, N, H, 64).float()
        k = y[..., lay.k_off:lay.k_off + H * 64].reshape(B, N, H, 64).float()
        iq = y[..., lay.iq_off:lay.iq_off + Hi * 64].reshape(B, N, Hi, 64).float()
        ik = y[..., lay.ik_off:lay.ik_off + Hi * 64].reshape(B, N, Hi, 64).float()
        q = F.layer_norm(q, (64,), norms[0][0], norms[0][1], 1e-5)
        k = F.layer_norm(k, (64,), norms[1][0], norms[1][1], 1e-5)
        ik = F.layer_norm(ik, (64,), norms[2][0], norms[2][1], 1e-5)
        outs = [rope_torch(t, pos).to(torch.bfloat16).contiguous() for t in (q, k, iq, ik)]
        return outs + [y[..., lay.iw_off:lay.iw_off + Hi].contiguous()]

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(steps)]
    for i in range(steps):
        one(evs[i])
    torch.cuda.synchronize()
    ph = [statistics.mean(e[j].elapsed_time(e[j + 1]) for e in evs) for j in range(5)]
    y = F.linear(x, w, b)
    for _ in range(warmup):
        torch_glue(y)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        torch_glue(y)
    e1.record(stream)
    torch.cuda.synchronize()
    torch_glue_ms = e0.elapsed_time(e1) / steps
    H, Hi = lay.H, lay.Hi
    glue_bytes = B * N * ((2 * H + 2 * Hi) * 64 + Hi) * 2 * 2 + B * N * 8
    return {
        "workload": f"whole sparse global-attention layer forward: B={B}, S={views} views (N={N}), dim {dim}, "
                    f"H={H}, indexer {Hi}x64, top-k {topk}, bf16, random-init weights",
        "value_ms": round(sum(ph), 3),
        "proj_gemm_ms": round(ph[0], 3),
        "glue_ms": round(ph[1], 3),
        "glue_gbs": round(glue_bytes / (ph[1] * 1e-3) / 1e9, 1),
        "indexer_ms": round(ph[2], 3),
        "attn_fwd_ms": round(ph[3], 3),
        "out_proj_ms": round(ph[4], 3),
        "torch_glue_ms": round(torch_glue_ms, 3),
    }


def layer_train_c4(steps: int = 3, warmup: int = 1, views: int = 24, batch: int = 2, topk: int = 1024):
    """The whole layer trained at the C4 shape (B=2, S=24 views, N=32,976), random-init
    weights, bf16: ``SparseGlobalAttention.forward_train`` (fused projection, glue, indexer
    top-k with scores, attention with attn_sum, output projection), the indexer KL loss on
    the normalised attention mass (detached, as the reference presets' detach_input), and the
    backward through every stage (GEMMs, glue, attention, indexer, KL). HIP events on the
    launch stream."""
    import torch

    from geoweave_amd import dsa_layer, workloads
    from geoweave_amd.custom_indexer import sparse_indexer_kl_loss

    dev = torch.device("cuda", 0)
    m = workloads.init_layer_(dsa_layer.SparseGlobalAttention(topk=topk)).to(dev).to(torch.bfloat16)
    x, pos = workloads.layer_module_inputs(views, batch)
    x, pos = x.to(dev).requires_grad_(), pos.to(dev)
    g = torch.Generator(device=dev).manual_seed(views)
    G = torch.randn(x.shape, generator=g, device=dev, dtype=torch.bfloat16)
    rope_len = int(pos.max()) + 1
    stream = torch.cuda.current_stream(dev)

    def one(ev=None):
        rec = (lambda i: ev[i].record(stream)) if ev else (lambda i: None)
        m.zero_grad(set_to_none=True)
        x.grad = None
        rec(0)
        out, attn, scores, _ = m.forward_train(x, pos, rope_len=rope_len)
        p = attn.detach().to(torch.bfloat16)
        p = p / (p.sum(-1, keepdim=True) + 1e-6)
        kl = sparse_indexer_kl_loss(p, scores, 1e-6)
        rec(1)
        torch.autograd.backward([out, kl], [G, None])
        rec(2)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(steps):
        one(evs[i])
    torch.cuda.synchronize()
    fwd = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    bwd = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)
    return {
        "workload": f"whole-layer training step: B={batch}, S={views} views (N={x.shape[1]}), dim 1024, 16 heads, "
                    f"indexer 4x64, top-k {topk}, bf16, random-init weights, output-gradient + indexer KL loss on the "
                    "detached attention mass",
        "fwd_ms": round(fwd, 3),
        "bwd_ms": round(bwd, 3),
        "step_ms": round(fwd + bwd, 3),
    }


def source_downsample_s32(qi, ki, wi, views: int, topk: int, steps: int = 10, warmup: int = 2):
    """The approximate coarse selector (source downsample, factor 2, inference only) on the
    metric's S=32 indexer inputs: pooled keys, indexer top-k over the 12,864 source rows and
    the expansion to top-k fine tokens, timed with HIP events. Not part of the metric (the
    metric is the exact top-k); reported so the approximate mode's cost is on record."""
    import torch

    from geoweave_amd import source_downsample as sd

    cfg = sd.SourceDownsample(tokens_per_view=qi.shape[1] // views, num_views=views, patch_start_idx=5, factor=2)
    layout = sd.build_layout(cfg)
    stream = torch.cuda.current_stream(qi.device)
    for _ in range(warmup):
        sd.select_topk(qi, ki, wi, topk, 0.125, cfg)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        sd.select_topk(qi, ki, wi, topk, 0.125, cfg)
    e1.record(stream)
    torch.cuda.synchronize()
    return {
        "workload": f"approximate top-{topk} by source downsample (factor 2): S={views} views, "
                    f"{qi.shape[1]} queries x {layout.source_len} source rows, then expansion",
        "select_ms": round(e0.elapsed_time(e1) / steps, 3),
        "source_rows": layout.source_len,
        "coarse_topk": sd.coarse_budget(layout, topk, cfg),
    }


def aggregator_c5(steps: int = 2, warmup: int = 1, views: int = 32, topk: int = 1024):
    """Config C5: the VGGT-1B-style aggregator forward (DINOv2-style ViT-L/14 patch
    embedding, 24 frame + 24 global blocks, dim 1024, 16 heads, MLP ratio 4, global blocks
    9-19 sparse with top-k 1024), random-init weights, bf16, S=32 seeded 518 x 518 images.
    Reports end-to-end latency (eager and replayed as one HIP graph) and the time inside the
    sparse global attention calls (HIP events around each call)."""
    import torch

    from geoweave_amd import aggregator as agg

    dev = torch.device("cuda", 0)
    with torch.device(dev):
        m = agg.Aggregator(indexer_layers="9-19", topk=topk)
    m = agg.random_init_(m, 20261201).to(torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(20261201 + views)
    images = torch.rand(1, views, 3, 518, 518, generator=g, device=dev)
    stream = torch.cuda.current_stream(dev)
    sparse_blocks = [b for b in m.global_blocks if b.sparse]

    for _ in range(warmup):
        m(images)
    torch.cuda.synchronize()
    e2e, sparse_ms = [], []
    for _ in range(steps):
        for b in sparse_blocks:
            b.timing = []
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        m(images)
        e1.record(stream)
        torch.cuda.synchronize()
        e2e.append(e0.elapsed_time(e1))
        sparse_ms.append(sum(a.elapsed_time(b) for blk in sparse_blocks for a, b in blk.timing))
    for b in sparse_blocks:
        b.timing = None
    graph = agg.AggregatorGraph(m)
    graph(images)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        graph(images)
    e1.record(stream)
    torch.cuda.synchronize()
    graph_ms = e0.elapsed_time(e1) / steps
    n_params = sum(p.numel() for p in m.parameters())
    e2e_ms, sp_ms = statistics.mean(e2e), statistics.mean(sparse_ms)
    return {
        "workload": f"C5 VGGT-1B-style aggregator forward: S={views} views of 518x518, 24 frame + 24 global blocks, "
                    f"dim 1024, 16 heads, global blocks 9-19 sparse (top-k {topk}), ViT-L/14 patch embedding, "
                    f"{n_params / 1e9:.2f} B random-init parameters, bf16",
        "e2e_ms": round(e2e_ms, 2),
        "e2e_graph_ms": round(graph_ms, 2),
        "sparse_global_attention_ms": round(sp_ms, 2),
        "sparse_global_attention_share": round(sp_ms / e2e_ms, 4),
    }


def cpu_model() -> str:
    """The host CPU's model name (``/proc/cpuinfo``), or the platform's fallback."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _oracle_layer(qi, ki, wi, q, k, v, rows, topk=1024):
    """(indexer s, attention s) of the fp32 CPU oracle on the given query rows."""
    from oracle import attention as oatt
    from oracle import indexer as oidx

    t0 = time.perf_counter()
    idx, _ = oidx.indexer_topk(qi[:, rows], ki, wi, None, topk, 0.125)
    t1 = time.perf_counter()
    oatt.sparse_attention(q[:, rows], k, v, idx, 0.125)
    t2 = time.perf_counter()
    return t1 - t0, t2 - t1


def cpu_baseline(views: int, sample_rows: int = 2048, runs: int = 3, c1_gpu_ms=None):
    """The fp32 CPU oracle (the restatement of the reference's torch backend: indexer scores
    + torch.topk + the gathered sparse attention) on the host cores.

    * ``value``: the metric's workload (S = ``views``) on a fixed sample of ``sample_rows``
      random query rows against all keys, median of ``runs`` passes after a warm-up pass,
      scaled to all rows (per-row cost does not depend on which rows).
    * ``c1_full``: config C1 (S = 4, N = 5,496) over every row, median of ``runs`` runs
      after a warm-up run, the indexer and the attention timed separately, beside the GPU's
      time for the same C1 step."""
    import torch

    from geoweave_amd import workloads

    torch.set_num_threads(os.cpu_count() or 1)
    lay = workloads.layer_inputs(views, 1, torch.bfloat16)
    t = [x.float() for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v)]
    n = lay.tokens
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(0))[:sample_rows]
    _oracle_layer(*t, rows)
    passes = [_oracle_layer(*t, rows) for _ in range(runs)]
    scale = n / rows.numel()
    med = sorted(passes, key=sum)[len(passes) // 2]
    del lay, t
    c1 = workloads.layer_inputs(4, 1, torch.bfloat16)
    t = [x.float() for x in (c1.q_idx, c1.k_idx, c1.w_idx, c1.q, c1.k, c1.v)]
    all_rows = torch.arange(c1.tokens)
    _oracle_layer(*t, all_rows)
    c1_runs = [_oracle_layer(*t, all_rows) for _ in range(runs)]
    c1_med = sorted(c1_runs, key=sum)[len(c1_runs) // 2]
    c1_ms = sum(c1_med) * 1e3
    return {
        "value": round(sum(med) * scale * 1e3, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"fp32 CPU oracle (indexer scores + torch.topk + gathered sparse attention) on a fixed "
                   f"sample of {rows.numel()} random query rows of the S={views} layer against all {n} keys, "
                   f"median of {runs} passes after a warm-up ({sum(med):.1f} s), scaled x{scale:.2f} to all rows"),
        "indexer_ms": round(med[0] * scale * 1e3, 1),
        "attn_fwd_ms": round(med[1] * scale * 1e3, 1),
        "cpu_model": cpu_model(),
        "c1_full": {
            "workload": f"C1: B=1, S=4 views (N={c1.tokens}), every query row, fp32, top-k 1024",
            "runs_ms": [round(sum(r) * 1e3, 1) for r in c1_runs],
            "median_ms": round(c1_ms, 1),
            "indexer_ms": round(c1_med[0] * 1e3, 1),
            "attn_fwd_ms": round(c1_med[1] * 1e3, 1),
            "gpu_ms": c1_gpu_ms,
            "cpu_over_gpu": None if not c1_gpu_ms else round(c1_ms / c1_gpu_ms, 1),
        },
    }


def gpu_step_ms(views: int, topk: int = 1024, steps: int = 10, warmup: int = 3) -> float:
    """GPU time of one metric step (indexer top-k + inference attention) at S = ``views``
    (HIP events on the launch stream, mean over ``steps``)."""
    import torch

    from geoweave_amd import workloads
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import sparse_index_flash_attn_inference_func
    from geoweave_amd.custom_indexer import sparse_topk_indexer_inference_func

    dev = torch.device("cuda", 0)
    lay = workloads.layer_inputs(views, 1, torch.bfloat16)
    qi, ki, wi, q, k, v = (x.to(dev) for x in (lay.q_idx, lay.k_idx, lay.w_idx, lay.q, lay.k, lay.v))
    stream = torch.cuda.current_stream(dev)

    def step():
        idx, _ = sparse_topk_indexer_inference_func(qi, ki, wi, qi.new_empty(0), topk, 0.125, 256, 0)
        sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=0.125)

    for _ in range(warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    return round(e0.elapsed_time(e1) / steps, 3)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--views", type=int, default=32)
    ap.add_argument("--topk", type=int, default=1024)
    ap.add_argument("--cpu-sample-rows", type=int, default=2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--with-attn-sum", action="store_true",
                    help="also time the training forward that writes attn_sum")
    ap.add_argument("--no-train", action="store_true", help="skip the C4 training-step timing")
    ap.add_argument("--no-long", action="store_true", help="skip the C3 (S=64) long-context timing")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-layer (projection + glue) timing")
    ap.add_argument("--no-c5", action="store_true", help="skip the C5 (full aggregator) timing")
    ap.add_argument("--no-sd", action="store_true", help="skip the approximate (source-downsample) top-k timing")
    ap.add_argument("--attn-path", choices=("auto", "dense", "gather"), default="auto",
                    help="attention forward without attn_sum: the masked dense pass, the gather kernel, "
                         "or the automatic choice (dense when S <= 96 K)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 3 plain device copies of 1 GiB (reference kernel for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE scaling)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the sparse global-attention path is benchmarked "
              "per GPU (queries shard across GPUs with one all-gather of K/V per layer, which "
              "this build does not launch). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from geoweave_amd import workloads
    from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import (
        sparse_index_flash_attn_inference_func,
    )
    from geoweave_amd.custom_flash_attn import sparse_index_flash_attn as sifa
    from geoweave_amd.custom_indexer import sparse_topk_indexer_inference_func

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 2
    sifa.FORWARD_PATH = args.attn_path
    dev = torch.device("cuda", 0)
    props = torch.cuda.get_device_properties(dev)

    views, topk = args.views, args.topk
    print(f"[bench] generating S={views} inputs", file=sys.stderr, flush=True)
    lay = workloads.layer_inputs(views, 1, torch.bfloat16)
    qi, ki, wi = (x.to(dev) for x in (lay.q_idx, lay.k_idx, lay.w_idx))
    q, k, v = (x.to(dev) for x in (lay.q, lay.k, lay.v))
    B, T, H, D = q.shape
    Hi, Di = qi.shape[2], qi.shape[3]
    empty_mask = qi.new_empty(0)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        idx, _ = sparse_topk_indexer_inference_func(qi, ki, wi, empty_mask, topk, 0.125, 256, 0,
                                                    return_scores=True)
        if ev is not None:
            ev[1].record(stream)
        o, _ = sparse_index_flash_attn_inference_func(q, k, v, idx, softmax_scale=0.125)
        if ev is not None:
            ev[2].record(stream)
        return idx, o

    print("[bench] warmup", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(args.steps):
        idx, o = step(evs[i])
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    idx_ms = [e[0].elapsed_time(e[1]) for e in evs]
    att_ms = [e[1].elapsed_time(e[2]) for e in evs]
    print(f"[bench] timed {args.steps} steps: {total_ms / args.steps:.3f} ms/step", file=sys.stderr, flush=True)

    Kk = idx.shape[-1]
    att_bytes = attn_fwd_algorithmic_bytes(B, T, H, D, Kk)
    idx_flops = indexer_algorithmic_flops(B, T, T, Hi, Di)
    att_avg = statistics.mean(att_ms)
    idx_avg = statistics.mean(idx_ms)
    att_gbs = att_bytes / (att_avg * 1e-3) / 1e9
    dense_flops = attn_fwd_dense_flops(B, T, T, H, D)
    dense_tflops = dense_flops / (att_avg * 1e-3) / 1e12
    idx_tflops = idx_flops / (idx_avg * 1e-3) / 1e12
    dense_used = sifa._use_dense(T, Kk, H, D)
    prof_name = f"dense_attn_fwd_S{views}_pmc.md" if dense_used else f"sparse_attn_fwd_S{views}_pmc.md"
    traffic = read_traffic_summary(REPO / "profiles" / prof_name)

    extra = {}
    if args.with_attn_sum:
        from geoweave_amd.custom_flash_attn.sparse_index_flash_attn import _flash_attn_forward

        for _ in range(2):
            _flash_attn_forward(q, k, v, idx, softmax_scale=0.125, return_attn=True)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(5):
            _flash_attn_forward(q, k, v, idx, softmax_scale=0.125, return_attn=True)
        e1.record(stream)
        torch.cuda.synchronize()
        extra["attn_fwd_with_attn_sum_ms"] = round(e0.elapsed_time(e1) / 5, 3)

    result = {
        "metric": METRIC,
        "value": round(total_ms / args.steps, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) attention q/k/v; indexer q/k/w from random projections)",
        "config": {
            "workload": f"one sparse global-attention layer fwd: indexer score + exact top-{topk} "
                        f"then sparse-index attention over the selected keys",
            "batch": B, "views": views, "tokens": T, "heads": H, "head_dim": D,
            "indexer_heads": Hi, "indexer_dim": Di, "topk": Kk,
        },
        "indexer_ms": round(idx_avg, 3),
        "attn_fwd_ms": round(att_avg, 3),
        "attn_path": "dense" if dense_used else "gather",
        # The roofline of what runs: the masked dense pass is bound by the matrix cores on
        # the flops it executes; the gather kernel by HBM on the bytes it gathers.
        "roofline": ({
            "kernel": "dense_attn_kernel (one attention call: + dense_mask_kernel, dense_vmax_kernel, "
                      "dense_vt_kernel)",
            "bound": "mfma",
            "achieved": round(dense_tflops, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(dense_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "algorithmic_flops": dense_flops,
        } if dense_used else {
            "kernel": "sparse_attn_fwd_kernel",
            "bound": "hbm",
            "achieved": round(att_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(att_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": att_bytes,
        }),
        # The sparse formulation's bytes (the selected K/V rows the reference gathers) over
        # the call's time: an effective rate of the whole attention, not a roofline of the
        # dense pass (which does not move these bytes).
        "attn_effective_gathered_bandwidth": {
            "gathered_bytes": att_bytes,
            "achieved": round(att_gbs, 1),
            "unit": "GB/s",
            "vs_hbm_peak": round(att_gbs / HBM_PEAK_GBS, 4),
        },
        "roofline_indexer": {
            "kernels": "indexer_score_kernel<sample>+select<tau>+score<filter>+select<final>+fallback",
            "bound": "mfma",
            "achieved": round(idx_tflops, 2),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(idx_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "algorithmic_flops": idx_flops,
        },
        "device": {"name": torch.cuda.get_device_name(dev), "arch": props.gcnArchName,
                   "cus": props.multi_processor_count},
        "timing": "HIP events on the launch stream; steady state, caches not flushed",
    }
    result.update(extra)
    if not args.no_sd:
        print("[bench] source-downsample selector", file=sys.stderr, flush=True)
        result["approx_topk_s32"] = source_downsample_s32(qi, ki, wi, views, topk)
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_layer:
        print("[bench] whole layer forward", file=sys.stderr, flush=True)
        result["layer_fwd_s32"] = layer_forward_s32()
    if not args.no_train:
        print("[bench] whole-layer training step", file=sys.stderr, flush=True)
        result["layer_train_c4"] = layer_train_c4()
    if not args.no_c5:
        print("[bench] C5 aggregator", file=sys.stderr, flush=True)
        result["aggregator_c5"] = aggregator_c5()
    if not args.no_long:
        print("[bench] C3 long context", file=sys.stderr, flush=True)
        result["long_context_c3"] = long_context_c3()
        torch.cuda.empty_cache()
    if not args.no_train:
        del idx, o
        print("[bench] C4 training step", file=sys.stderr, flush=True)
        result["train_c4"] = train_step_c4()
    if not args.no_cpu_baseline:
        del lay
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        c1_gpu = gpu_step_ms(4, topk)
        result["cpu_baseline"] = cpu_baseline(views, args.cpu_sample_rows, c1_gpu_ms=c1_gpu)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
