#!/usr/bin/env python3
"""Benchmark of the GRPO rollout-and-loss hot path on one MI355X.

Headline (``value``): paged decode attention HBM GB/s for one full decode
step of Qwen3-0.6B at the serving shape -- 28 layers, 64 sequences with
contexts ~ U{1024..4096}, 16 query / 8 KV heads, head_dim 128, 256-token
pages with shuffled block tables.  Each layer owns its own K/V pool (18.8 GB
in total), so the 256 MB Infinity Cache cannot serve the reads.  A "step" is
the 28 decode-attention launches of one decode step, captured in one HIP graph
as the engine runs them; ``roofline.achieved`` comes from per-launch events.

Secondary legs (same JSON line): the fused GRPO logprob+advantage+loss kernel
on the 32x512x151936 loss step, the KV store at 65,536 tokens, the varlen
paged prefill on the prefix-cache chunk workload (MFMA TFLOP/s), and the CPU
oracle (the CPU restatement of the reference semantics) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--legs decode1,decode,grpo,store,prefill,norm_rope,host,rollout]
       [--no-cpu] [--calibrate-copy]
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# HBM bytes per decode launch (balanced split + merge) at the 28-layer B=64 shape,
# measured by two rocprofv3 --pmc passes (FETCH_SIZE scaled by 2.0, WRITE_SIZE by
# 1.0, the factors a plain copy of known size gives); recorded in
# profiles/paged_decode_28layer_b64_ctx1024-4096.md.
DECODE_TRAFFIC_BYTES = 671878759
METRIC = "decode-attn HBM GB/s (% of 8 TB/s); GRPO rollout tokens/s on 1 GPU"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_pkg():
    lib = ROOT / "qwen3-naive-inference_amd" / "libqwen3mi.so"
    if not lib.exists():
        importlib.import_module("__graft_entry__").build()
    return importlib.import_module("qwen3-naive-inference_amd")


def warm_up(torch, fn_list, seconds):
    """Run fn_list repeatedly for about ``seconds`` (untimed), so that a leg
    that follows a CPU-only phase is timed at the GPU's running clocks."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for fn in fn_list:
            fn()
        torch.cuda.synchronize()


def timed_launches(torch, fn_list, steps, warmup):
    """Run ``warmup`` untimed steps, then ``steps`` timed steps.

    Each step calls every function in ``fn_list`` once.  Returns (total ms
    for the timed steps, list of per-call ms from events bracketing each call
    on the launch stream).
    """
    for _ in range(warmup):
        for fn in fn_list:
            fn()
    torch.cuda.synchronize()
    n = steps * len(fn_list)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    k = 0
    for _ in range(steps):
        for fn in fn_list:
            starts[k].record()
            fn()
            ends[k].record()
            k += 1
    t1.record()
    torch.cuda.synchronize()
    total = t0.elapsed_time(t1)
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return total, per


def graph_us_per_call(torch, fn, steps, warmup, per_graph=20):
    """GPU µs per call of ``fn``: ``per_graph`` calls captured in one HIP graph,
    replayed; for launches shorter than the host-side cost of a call."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            fn()
    reps = max(2, steps // 2)
    total_ms, _ = timed_launches(torch, [graph.replay], reps, max(1, warmup))
    return total_ms * 1e3 / (reps * per_graph)


# ---------------------------------------------------------------------------
def leg_decode(torch, pkg, W, dev, steps, warmup, layers=28):
    log(f"decode: generating {layers}-layer pools (B=64, ctx U[1024,4096])")
    w = W.decode_batch(seed=0, device=dev, batch=64, layers=layers)
    q, kc, vc = w["q"], w["k_cache"], w["v_cache"]
    lens, bt, scale = w["cache_seqlens"], w["block_tables"], w["scale"]
    out = torch.empty_like(q)
    kv_bytes = W.decode_kv_bytes(lens.cpu())
    other = q.numel() * 2 + out.numel() * 2 + bt.numel() * 4 + lens.numel() * 4
    per_launch_bytes = kv_bytes + other

    fns = [(lambda l=l: pkg.kernels.paged_decode_attention(q, kc[l], vc[l], lens, bt, scale,
                                                           out=out)) for l in range(layers)]
    log("decode: timing")
    total_ms, per = timed_launches(torch, fns, steps, warmup)
    eager_ms_step = total_ms / steps
    avg_launch_ms = statistics.mean(per)
    # The step as the engine runs it: the 28 launches captured in one HIP graph
    # (no host work or events between launches), replayed back to back.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fns:
            fn()
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps
    del graph
    gbs_step = per_launch_bytes * layers / (ms_step * 1e-3) / 1e9
    gbs_launch = per_launch_bytes / (avg_launch_ms * 1e-3) / 1e9
    return dict(ms_per_step=ms_step, eager_ms_per_step=eager_ms_step, gbs=gbs_step,
                avg_launch_us=avg_launch_ms * 1e3,
                launch_gbs=gbs_launch, bytes_per_launch=per_launch_bytes,
                kv_bytes_per_launch=kv_bytes, layers=layers,
                mean_ctx=float(lens.float().mean().item() - 1),
                workload=w)


def init_qwen3_weights(torch, model, std=0.02):
    """Random init as transformers initialises Qwen3: N(0, std) matrices and
    embedding (tied lm_head), unit norm weights."""
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            else:
                p.normal_(0.0, std)


def make_qwen3(torch, pkg, dev, seed=0):
    torch.manual_seed(seed)
    with torch.device(dev):
        model = pkg.Qwen3ForCausalLM(pkg.Qwen3Config())
    init_qwen3_weights(torch, model)
    return model.to(torch.bfloat16).eval()


def leg_decode_step(torch, pkg, dev, steps, warmup, w, attn_ms_step):
    """Config 3 as a whole: one 28-layer Qwen3-0.6B decode step for the
    64-sequence serving batch (embedding, per layer add+RMSNorm, qkv GEMM,
    paged attention with the QK-norm/RoPE/KV store folded in, o GEMM, add+RMSNorm,
    gate_up GEMM, SwiGLU, down GEMM; final norm), captured as the engine's
    HIP graph and replayed; then the lm_head and the fused sampler.  Uses the
    decode leg's 28-layer pools, contexts and page tables (``w``)."""
    log("decode_step: 28-layer model on the decode leg's pools")
    model = make_qwen3(torch, pkg, dev)
    for i, layer in enumerate(model.model.layers):
        layer.self_attn.k_cache = w["k_cache"][i]
        layer.self_attn.v_cache = w["v_cache"][i]
    model._num_blocks = w["num_blocks"]
    ctx, bt = w["context_lens"], w["block_tables"]
    bsz = ctx.shape[0]
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 151936, (bsz,), generator=g).to(dev)
    pos = ctx.long()
    slots = (bt.long().gather(1, (pos // 256)[:, None])[:, 0] * 256 + pos % 256).to(torch.int32)
    with torch.no_grad():
        model._init_cuda_graphs(max_bs=bsz, bt_width=bt.shape[1])
        model._capture_decode_graphs(batch_sizes=(bsz,))
        assert model._has_cuda_graphs, "decode graph capture failed"
        bufs = model._graph_bufs
        bufs["input_ids"][:bsz] = ids
        bufs["positions"][:bsz] = pos
        bufs["slot_mapping"][:bsz] = slots
        bufs["context_lens"][:bsz] = ctx
        bufs["block_tables"][:bsz] = bt
        graph = model._graphs[bsz]
        h = bufs["outputs"][:bsz]
        body_ms, _ = timed_launches(torch, [graph.replay], steps, warmup)
        body_ms /= steps

        def head():  # the engine's head: fused lm_head + sampling (top_k=None)
            return model._sample(h, 1.0, None, True)
        full_ms, _ = timed_launches(torch, [lambda: (graph.replay(), head())], steps, warmup)
        full_ms /= steps
        lm_ms, _ = timed_launches(torch, [lambda: model.lm_head(h)], steps, warmup)
        lm_ms /= steps  # the unfused [B, V] lm_head GEMM alone, for comparison
    weights = sum(p.numel() * 2 for p in model.parameters())
    kv = W_kv_bytes(w)
    out = dict(ms_per_step=body_ms, ms_per_step_with_lm_head_and_sampling=full_ms,
               unfused_lm_head_gemm_ms=lm_ms, attention_ms_per_step=attn_ms_step,
               attention_share=attn_ms_step / body_ms, batch=bsz,
               weight_bytes=weights, kv_bytes_per_step=kv,
               hbm_gbs=(kv + weights) / (body_ms * 1e-3) / 1e9)
    model._graphs, model._graphs_units, model._graph_bufs, model._graph_pool = {}, {}, None, None
    for layer in model.model.layers:
        layer.self_attn.k_cache = layer.self_attn.v_cache = None
    del model, graph, h
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def leg_decode_step256(torch, pkg, dev, steps, warmup, ctx_len=640, bsz=256):
    """The rollout's decode step: 256 sequences at the rollout's mean context
    (640 cached keys; all sequences of a rollout step have near-equal contexts),
    the 28-layer model with one K/V page pool slice per layer as the engine
    allocates it, replayed through the engine's own decode path
    (``_run_decode_graph_seqs``: one host-to-device copy of the step's inputs,
    then the whole-unit graph of the 256-row bucket); then with the fused
    lm_head + sampler (all entries, and the top 20)."""
    log(f"decode_step256: {bsz} sequences x {ctx_len} keys, 28 layers")
    model = make_qwen3(torch, pkg, dev)
    pages = bsz * ((ctx_len + 1 + 255) // 256) + 2
    model.allocate_global_kv_cache(num_blocks=pages)
    for layer in model.model.layers:
        layer.self_attn.k_cache.normal_()
        layer.self_attn.v_cache.normal_()
    model._ensure_engine(True, bt_width=(ctx_len + 1 + 255) // 256)
    bm = pkg.BlockManager(pages)
    g = torch.Generator().manual_seed(1)
    seqs = []
    for _ in range(bsz):
        s = pkg.Sequence(torch.randint(0, 151936, (ctx_len + 1,), generator=g).tolist())
        bm.allocate(s)
        s.kv_len = ctx_len
        s.num_scheduled_tokens = 1
        seqs.append(s)
    model.last_stats = {}
    with torch.no_grad():
        step = lambda: model._run_decode_graph_seqs(seqs)
        body_ms, _ = timed_launches(torch, [step], steps, warmup)
        body_ms /= steps
        unit_graph = model.last_stats.get("unit_graph_steps", 0) > 0
        h = step()
        rec = {}
        for name, k in (("sample", None), ("topk20", 20)):
            ms, _ = timed_launches(torch, [lambda: (step(), model._sample(h, 1.0, k, True))],
                                   steps, warmup)
            rec[f"ms_per_step_with_lm_head_and_{name}"] = ms / steps
    kv = 28 * bsz * (ctx_len + 1) * 8 * 128 * 2 * 2
    weights = sum(p.numel() * 2 for p in model.parameters())
    out = dict(ms_per_step=body_ms, us_per_layer=body_ms * 1e3 / 28, batch=bsz,
               context=ctx_len, whole_unit_graph=unit_graph, kv_bytes_per_step=kv,
               weight_bytes=weights, hbm_gbs=(kv + weights) / (body_ms * 1e-3) / 1e9, **rec)
    model._graphs, model._graphs_units, model._graph_bufs, model._graph_pool = {}, {}, None, None
    for layer in model.model.layers:
        layer.self_attn.k_cache = layer.self_attn.v_cache = None
    del model, h
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def W_kv_bytes(w) -> int:
    """K/V bytes a 28-layer decode step reads (ctx + 1 keys per sequence and layer)."""
    return int(w["k_cache"].shape[0]) * int(w["kv_bytes"])


def leg_lm_head(torch, pkg, dev, steps, warmup, vocab=151936, hidden=1024):
    """Fused lm_head + sampling (rollout decode rows) and fused lm_head +
    log-prob gather (loss-step rows) against the unfused pair they replace
    (hipBLASLt logits GEMM, then the streaming sampler / log-prob kernel)."""
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    w = (0.02 * torch.randn((vocab, hidden), generator=g, device=dev)).to(torch.bfloat16)
    out = {}
    wbytes = vocab * hidden * 2
    for n in (64, 256):
        h = torch.randn((n, hidden), generator=g, device=dev).to(torch.bfloat16)
        fused = lambda: pkg.kernels.lm_head_sample(h, w, 1.0, seed=1, offset=2)
        unfused = lambda: pkg.kernels.sample_tokens(h @ w.T, 1.0, seed=1, offset=2)
        gemm = lambda: h @ w.T
        rec = {}
        for name, fn in (("fused_us", fused), ("unfused_us", unfused), ("gemm_only_us", gemm)):
            _, per = timed_launches(torch, [fn], steps, warmup)
            rec[name] = round(statistics.median(per) * 1e3, 2)
        flops = 2 * n * hidden * vocab
        t = rec["fused_us"] * 1e-6
        rec.update(rows=n, weight_bytes=wbytes, hbm_gbs=round(wbytes / t / 1e9, 1),
                   frac_of_hbm_peak=round(wbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                   tflops=round(flops / t / 1e12, 1),
                   frac_of_bf16_mfma_peak=round(flops / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4))
        out[f"sample_{n}_rows"] = rec
    # Top-k = 20 (the reference's default), at the rollout's 256 rows and
    # config 3's 64: the fused lm_head + top-k sampler (no logits), against
    # the materialised bf16 logits + the HIP radix-select sampler, and the
    # reference's torch ops on those logits.
    for n in (64, 256):
        h = torch.randn((n, hidden), generator=g, device=dev).to(torch.bfloat16)
        logits = h @ w.T

        def torch_topk():
            x = logits.float() / 0.6
            vals, idx = torch.topk(x, 20, dim=-1)
            x = torch.full_like(x, float("-inf")).scatter(-1, idx, vals)
            nxt = torch.multinomial(torch.softmax(x, dim=-1), num_samples=1)
            return nxt, torch.log_softmax(x, dim=-1).gather(-1, nxt)
        rec = {}
        for name, fn in (
                ("fused_us", lambda: pkg.kernels.lm_head_sample(h, w, 0.6, seed=1, top_k=20)),
                ("gemm_plus_hip_sampler_us",
                 lambda: pkg.kernels.sample_tokens_topk(h @ w.T, 20, 0.6, seed=1)),
                ("hip_sampler_only_us", lambda: pkg.kernels.sample_tokens_topk(logits, 20, 0.6,
                                                                               seed=1)),
                ("torch_ops_only_us", torch_topk)):
            _, per = timed_launches(torch, [fn], steps, warmup)
            rec[name] = round(statistics.median(per) * 1e3, 2)
        rec["rows"] = n
        out[f"topk20_sampling_{n}_rows"] = rec
        del logits
    n = 8192
    h = torch.randn((n, hidden), generator=g, device=dev).to(torch.bfloat16)
    tgt = torch.randint(0, vocab, (n,), generator=g, device=dev)
    fused = lambda: pkg.kernels.lm_head_logprob(h, w, tgt)
    unfused = lambda: pkg.kernels.logprob_gather(h @ w.T, tgt)
    rec = {}
    for name, fn in (("fused_us", fused), ("unfused_us", unfused)):
        _, per = timed_launches(torch, [fn], max(3, steps // 4), warmup)
        rec[name] = round(statistics.median(per) * 1e3, 1)
    flops = 2 * n * hidden * vocab
    rec.update(rows=n, tflops=round(flops / (rec["fused_us"] * 1e-6) / 1e12, 1),
               frac_of_bf16_mfma_peak=round(flops / (rec["fused_us"] * 1e-6) / 1e12 /
                                            MFMA_BF16_PEAK_TFLOPS, 4),
               logits_bytes_not_materialised=n * vocab * 2)
    out[f"logprob_{n}_rows"] = rec
    del w, h
    torch.cuda.empty_cache()
    return out


def leg_grpo(torch, pkg, W, dev, steps, warmup):
    log("grpo: generating 32x512x151936 bf16 logits")
    w = W.grpo_loss_step(seed=0, device=dev)
    args = (w["logits"], w["ids"], w["old_lp"], w["mask"], w["rewards"], w["prompt_ids"])
    fn = lambda: pkg.kernels.grpo_fused_forward(*args, 1e-4, 0.2, "seq")
    log("grpo: timing")
    total_ms, per = timed_launches(torch, [fn], steps, warmup)
    rows = 32 * 512
    nbytes = w["logit_bytes"] + rows * 8 + 2 * rows * 4 + 3 * rows * 4
    ms = statistics.mean(per)
    res = fn()
    torch.cuda.synchronize()
    out = dict(avg_launch_us=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, bytes_per_launch=nbytes,
               loss=float(res["loss"].item()))
    # Backward through the log-softmax (d loss / d logits, bf16): rows with a
    # non-zero coefficient read their logits, every row writes its gradient.
    log("grpo: backward timing")
    grad = torch.empty_like(w["logits"])
    lse, dlp = res["lse"], res["dlp"]
    gscale = torch.ones((), dtype=torch.float32, device=dev)
    bwd = lambda: pkg.kernels.logprob_gather_backward(w["logits"], w["ids"], lse, dlp,
                                                      grad_scale=gscale, out=grad)
    _, per_b = timed_launches(torch, [bwd], max(3, steps // 2), warmup)
    ms_b = statistics.mean(per_b)
    active = int((dlp != 0).sum().item())
    row_bytes = 151936 * 2
    b_bytes = active * row_bytes + rows * row_bytes + rows * (8 + 8)
    out.update(bwd_avg_launch_us=ms_b * 1e3, bwd_gbs=b_bytes / (ms_b * 1e-3) / 1e9,
               bwd_bytes_per_launch=b_bytes, bwd_active_rows=active)
    del w, args, res, grad
    torch.cuda.empty_cache()
    return out


def leg_store(torch, pkg, dev, steps, warmup, n_tok=65536, cpu=True, n_sets=4):
    """KV store of 65,536 tokens into a shuffled pool.  Launches rotate over
    ``n_sets`` independent (inputs, pool, slots) sets, 2.2 GB in all, so no
    launch finds its data in the 256 MB Infinity Cache."""
    log(f"store: {n_tok} tokens, {n_sets} rotating sets")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    nb = n_tok // 256 + 16
    sets = []
    for r in range(n_sets):
        key = torch.randn((n_tok, 8, 128), generator=g, device=dev).to(torch.bfloat16)
        val = torch.randn((n_tok, 8, 128), generator=g, device=dev).to(torch.bfloat16)
        kc = torch.empty((nb, 256, 8, 128), dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        gc = torch.Generator().manual_seed(r)
        slots = torch.randperm(nb * 256, generator=gc)[:n_tok].to(torch.int32).to(dev)
        sets.append((key, val, kc, vc, slots))
    fns = [(lambda s=s: pkg.kernels.store_kvcache(*s)) for s in sets]
    total_ms, per = timed_launches(torch, fns, steps, warmup)
    key, val, kc, vc, slots = sets[0]
    nbytes = 2 * 2 * key.numel() * 2 + slots.numel() * 4
    ms = statistics.mean(per)
    res = dict(avg_launch_us=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, bytes_per_launch=nbytes,
               tokens=n_tok, rotating_sets=n_sets)
    if cpu:
        # The oracle's per-token store (one row copy per token, as the reference
        # launches one program per token) on the host, over an 8,192-token sample.
        from oracle import paged as OP
        torch.set_num_threads(os.cpu_count() or 1)
        n_s = 8192
        k_c, v_c = key[:n_s].cpu(), val[:n_s].cpu()
        kc_c = torch.zeros((nb, 256, 8, 128), dtype=torch.bfloat16)
        vc_c = torch.zeros_like(kc_c)
        sl = slots[:n_s].cpu()
        times = []
        for _ in range(3):
            t = time.perf_counter()
            OP.store_kvcache(k_c, v_c, kc_c, vc_c, sl)
            times.append(time.perf_counter() - t)
        med = statistics.median(times)
        rows = kc.view(-1, 1024)[slots[:n_s].long()].cpu()
        res["rows_bit_exact_vs_oracle"] = bool(torch.equal(rows, kc_c.view(-1, 1024)[sl.long()]))
        res["cpu_baseline"] = dict(value=round(2 * 2 * n_s * 1024 * 2 / med / 1e9, 3), unit="GB/s",
                                   cores=torch.get_num_threads(), kind="port",
                                   sample=f"oracle store_kvcache (torch CPU, per-token loop), "
                                          f"{n_s} tokens", seconds_per_sample=med)
    return res


def leg_norm_rope(torch, pkg, dev, steps, warmup):
    """Fused per-head QK-RMSNorm + RoPE + KV store (one call per layer in the
    model) at a decode batch (256 tokens) and a prefill chunk (8,192 tokens):
    reads the qkv row (8 KB per token), its position, slot and cos/sin row
    (512 B), writes q (4 KB) and the K and V rows (2 KB each) of the token."""
    from oracle import norm_rope as ON
    from oracle import paged as OP
    qmod = pkg.qwen3_naive
    rope = qmod.RotaryEmbedding(128, 40960, 1000000.0)
    cache = rope.cos_sin_cache.to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    qw = (1.0 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1.0 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    out = {}
    per_token = 4096 * 2 + 2048 * 2 + 2 * 1024 * 2 + 8 + 4 + 128 * 4
    for name, n in (("decode_256", 256), ("prefill_8192", 8192)):
        nb = n // 256 + 8
        kc = torch.zeros((nb, 256, 8, 128), dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        qkv = torch.randn((n, 4096), generator=g, device=dev).to(torch.bfloat16)
        pos = torch.randint(0, 4096, (n,), generator=g, device=dev)
        gc = torch.Generator().manual_seed(n)
        slots = torch.randperm(nb * 256, generator=gc)[:n].to(torch.int32).to(dev)
        fn = lambda: pkg.kernels.qk_norm_rope_store(qkv, qw, kw, pos, cache, 16, 8, 1e-6, kc, vc,
                                                    slots)
        us = graph_us_per_call(torch, fn, steps, warmup)
        _, per = timed_launches(torch, [fn], max(10, steps // 2), warmup)
        q = fn()
        torch.cuda.synchronize()
        rec = dict(tokens=n, us_per_launch=round(us, 2),
                   us_per_eager_call=round(statistics.median(per) * 1e3, 2),
                   bytes_per_launch=per_token * n,
                   gbs=round(per_token * n / (us * 1e-6) / 1e9, 1))
        rec["frac_of_hbm_peak"] = round(rec["gbs"] / HBM_PEAK_GBS, 4)
        if name == "prefill_8192":
            # Oracle on the host: norm + rotate + store, fp32 math, bf16 results.
            torch.set_num_threads(os.cpu_count() or 1)
            qkv_c, pos_c, cache_c = qkv.cpu(), pos.cpu(), cache.cpu()
            kc_c, vc_c = torch.zeros_like(kc, device="cpu"), torch.zeros_like(vc, device="cpu")

            def cpu_step():
                qh = ON.rms_norm(qkv_c[:, :2048].reshape(n, 16, 128), qw.cpu(), 1e-6)
                kh = ON.rms_norm(qkv_c[:, 2048:3072].reshape(n, 8, 128), kw.cpu(), 1e-6)
                qr = ON.apply_rope(qh, pos_c, cache_c)
                kr = ON.apply_rope(kh, pos_c, cache_c)
                OP.store_kvcache(kr, qkv_c[:, 3072:].reshape(n, 8, 128), kc_c, vc_c, slots.cpu())
                return qr
            times = []
            for _ in range(3):
                t = time.perf_counter()
                q_ref = cpu_step()
                times.append(time.perf_counter() - t)
            med = statistics.median(times)
            rec["max_abs_err_q_vs_oracle"] = (q.float().cpu() - q_ref.float()).abs().max().item()
            rec["max_abs_err_k_rows_vs_oracle"] = (kc.float().cpu() - kc_c.float()).abs().max().item()
            rec["v_rows_bit_exact"] = bool(torch.equal(vc.cpu(), vc_c))
            rec["cpu_baseline"] = dict(value=round(per_token * n / med / 1e9, 3), unit="GB/s",
                                       cores=torch.get_num_threads(), kind="port",
                                       sample="oracle rms_norm + apply_rope + store_kvcache "
                                              "(fp32 torch CPU, per-token store loop), 8,192 tokens",
                                       seconds_per_sample=med)
        out[name] = rec
    # RMSNorm, residual add + RMSNorm and SwiGLU of the layer body over 8,192
    # token rows (hidden 1024, intermediate 3072), against the oracle.
    n = 8192
    x = torch.randn((n, 1024), generator=g, device=dev).to(torch.bfloat16)
    r = torch.randn((n, 1024), generator=g, device=dev).to(torch.bfloat16)
    wn = (1.0 + 0.1 * torch.randn(1024, generator=g, device=dev)).to(torch.bfloat16)
    gu = torch.randn((n, 6144), generator=g, device=dev).to(torch.bfloat16)
    body = {
        "rms_norm_8192x1024": (lambda: pkg.kernels.rms_norm(x, wn, 1e-6), n * 1024 * 2 * 2),
        "add_rms_norm_8192x1024": (lambda: pkg.kernels.add_rms_norm(x, r, wn, 1e-6),
                                   n * 1024 * 2 * 4),
        "silu_mul_8192x3072": (lambda: pkg.kernels.silu_mul(gu), n * 3072 * 2 * 3),
    }
    for name, (fn, nbytes) in body.items():
        us = graph_us_per_call(torch, fn, steps, warmup)
        rec = dict(us_per_launch=round(us, 2), bytes_per_launch=nbytes,
                   gbs=round(nbytes / (us * 1e-6) / 1e9, 1))
        rec["frac_of_hbm_peak"] = round(rec["gbs"] / HBM_PEAK_GBS, 4)
        out[name] = rec
    return out


def leg_host_prepare(torch, pkg, n_seqs=256, steps=200):
    """Host-side decode step preparation (slot of the new token, -1-padded
    page tables, ids, positions, context lengths) for 256 sequences of ~640
    tokens (3 pages), as numpy arrays ready for one pinned copy; beside it the
    oracle's per-sequence restatement of the reference's loops."""
    from oracle import paged as OP
    P = pkg.paged
    rng = __import__("random").Random(0)
    seqs, dicts = [], []
    for i in range(n_seqs):
        n_tok = 129 + rng.randrange(1024)
        s = P.Sequence([rng.randrange(151936) for _ in range(n_tok)])
        s.block_table = [rng.randrange(1362) for _ in range((n_tok + 255) // 256)]
        s.kv_len = n_tok - 1
        seqs.append(s)
        dicts.append(dict(block_table=s.block_table, kv_len=s.kv_len))
    P.prepare_decode(seqs)
    t = time.perf_counter()
    for _ in range(steps):
        P.prepare_decode(seqs)
    ours = (time.perf_counter() - t) / steps

    def oracle_step():
        slots = [OP.decode_slot(d["block_table"], d["kv_len"]) for d in dicts]
        tables = OP.block_tables([d["block_table"] for d in dicts])
        ids = [s.token_ids[-1] for s in seqs]
        pos = [len(s.token_ids) - 1 for s in seqs]
        ctx = [d["kv_len"] for d in dicts]
        return torch.tensor(ids), torch.tensor(pos), torch.tensor(ctx, dtype=torch.int32), \
            torch.tensor(tables, dtype=torch.int32), torch.tensor(slots, dtype=torch.int32)
    oracle_step()
    t = time.perf_counter()
    for _ in range(steps):
        oracle_step()
    ref = (time.perf_counter() - t) / steps
    got = P.prepare_decode(seqs)
    want = oracle_step()
    same = all(bool((torch.as_tensor(a).long() == b.long()).all()) for a, b in zip(got, want))
    return dict(sequences=n_seqs, us_per_step=round(ours * 1e6, 1),
                oracle_loop_us_per_step=round(ref * 1e6, 1), equal_to_oracle=same)


def leg_prefill(torch, pkg, W, dev, steps, warmup, cpu=True):
    """Config 4: one layer's attention over every chunk step of the prefix-cache
    workload (16 sequences, 512-token shared prefix, suffixes U{256..2048} in
    512-token chunks).  Algorithmic FLOPs count unmasked (query, key) pairs."""
    sched = W.prefix_prefill_chunks(seed=0)
    n_blocks = 2 + 16 * 16
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    kc = torch.randn((n_blocks, 256, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((n_blocks, 256, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    calls, pairs = [], 0
    for i, step in enumerate(sched["steps"]):
        inp = W.prefill_step_inputs(i, step, [0, 1], n_blocks, device=dev)
        pairs += W.causal_pairs(inp["cu_seqlens_q"].tolist(), inp["cu_seqlens_k"].tolist())
        calls.append(inp)
    flops = 4 * 16 * 128 * pairs
    fns = [(lambda c=c: pkg.kernels.varlen_prefill_attention(
        c["q"], kc, vc, c["cu_seqlens_q"], c["cu_seqlens_k"], c["max_seqlen_q"],
        c["max_seqlen_k"], 128 ** -0.5, True, c["block_tables"])) for c in calls]
    # The leg follows the KV-store leg's CPU baseline (the GPU idles for tens
    # of seconds): half a second of its own launches first.
    warm_up(torch, fns, 0.5)
    _, per = timed_launches(torch, fns, steps, warmup)
    # The layer's four launches back to back, with events only around the whole
    # timed region (events between launches add gaps the model does not have).
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        for fn in fns:
            fn()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    res = dict(ms_per_layer=ms, tflops=flops / (ms * 1e-3) / 1e12, flops=flops,
               causal_pairs=pairs, n_steps=len(calls),
               ms_per_layer_launch_events=sum(per) / steps,
               q_tokens=sum(int(c["cu_seqlens_q"][-1]) for c in calls))
    if cpu:
        # The oracle (fp32 torch CPU) on the first two sequences of the first
        # chunk step: 2 x 512 queries over 1,024 keys each.
        from oracle import attention as OA
        torch.set_num_threads(os.cpu_count() or 1)
        c = calls[0]
        cq = c["cu_seqlens_q"].cpu()[:3]
        ck = c["cu_seqlens_k"].cpu()[:3]
        nq = int(cq[-1])
        q_c = c["q"][:nq].cpu()
        bt_c = c["block_tables"][:2].cpu()
        kc_c, vc_c = kc.cpu(), vc.cpu()
        s_pairs = W.causal_pairs(cq.tolist(), ck.tolist())
        times = []
        for _ in range(2):
            t = time.perf_counter()
            ref = OA.varlen_prefill(q_c, kc_c, vc_c, cq, ck, bt_c, 128 ** -0.5)
            times.append(time.perf_counter() - t)
        med = statistics.median(times)
        out = fns[0]()
        torch.cuda.synchronize()
        res["max_abs_err_vs_oracle"] = (out[:nq].float().cpu() - ref).abs().max().item()
        res["cpu_baseline"] = dict(value=round(4 * 16 * 128 * s_pairs / med / 1e12, 4),
                                   unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                                   sample="oracle varlen_prefill (fp32 torch CPU), first two "
                                          "sequences of the first chunk step (2 x 512 queries)",
                                   seconds_per_sample=med)
    return res


# ---------------------------------------------------------------------------
# End-to-end GRPO rollout + loss (config 5) and the reference-path baseline.
class TorchBody:
    """Model body of the torch reference path: torch ops for RMSNorm, QK-norm,
    RoPE, SwiGLU and the KV store (index_copy_), and attention as torch SDPA
    over K/V gathered from the pages for the keys each sequence needs, padded
    to the step's longest sequence (flash-attn is not installed in this
    image).  The query heads of a KV head are folded into the query length, so
    no K/V copy is made per query head.  A mixed step runs its decode rows
    (one query) as one batch and its prefill rows as another.  Per-step
    metadata (host lengths, padded index maps) is built once per step, not per
    layer.  Bench-only: the product has one backend."""

    attention_kind = "torch SDPA (memory-efficient / flash backends, bf16)"

    def __init__(self, torch, pkg):
        self.torch, self.pkg = torch, pkg
        self.QN = pkg.qwen3_naive
        self._meta_key = None
        self._meta = None

    def _project(self, attn, x, positions):
        qkv = attn.qkv_proj(x)
        n = x.shape[0]
        q, k, v = qkv.split([attn.q_size, attn.kv_size, attn.kv_size], dim=-1)
        q = attn.q_norm(q.reshape(n, attn.num_heads, attn.head_dim))
        k = attn.k_norm(k.reshape(n, attn.num_kv_heads, attn.head_dim))
        cache = attn._cos_sin(x.device)
        rot = self.QN.RotaryEmbedding.rotate
        return (rot(q, positions, cache), rot(k, positions, cache),
                v.reshape(n, attn.num_kv_heads, attn.head_dim))

    def _store(self, attn, k, v, slots):
        row = attn.num_kv_heads * attn.head_dim
        idx = slots.long()
        attn.k_cache.view(-1, row).index_copy_(0, idx, k.reshape(-1, row))
        attn.v_cache.view(-1, row).index_copy_(0, idx, v.reshape(-1, row))

    def _sdpa(self, q, k, v, mask):
        t = self.torch
        from torch.nn.attention import SDPBackend, sdpa_kernel
        if TorchBody.attention_kind.startswith("torch SDPA"):
            try:
                with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]):
                    return t.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
            except RuntimeError:
                TorchBody.attention_kind = "fp32 matmul attention (no fused SDPA kernel)"
        # fp32 products: batched bf16 products with transposed operands are
        # avoided on this platform.
        s = t.matmul(q.float(), k.float().transpose(-2, -1).contiguous()) * q.shape[-1] ** -0.5
        s = s.masked_fill(~mask, float("-inf"))
        return t.matmul(t.softmax(s, -1), v.float()).to(q.dtype)

    def _gather_kv(self, attn, slots):
        """K and V rows at slots [B, L] -> [B, Hkv, L, D] views."""
        hkv, d = attn.num_kv_heads, attn.head_dim
        kk = attn.k_cache.view(-1, hkv, d)[slots].transpose(1, 2)
        vv = attn.v_cache.view(-1, hkv, d)[slots].transpose(1, 2)
        return kk, vv

    def _attend(self, attn, q, slots, mask, lq):
        """q [B, lq, Hq, D], key slots [B, L], mask [B, lq, L] -> [B, lq, Hq, D]."""
        bsz = q.shape[0]
        hkv, d = attn.num_kv_heads, attn.head_dim
        rep = attn.num_heads // hkv
        kk, vv = self._gather_kv(attn, slots)
        # query head h -> KV head h // rep: fold (rep, lq) into the query axis
        qg = q.view(bsz, lq, hkv, rep, d).permute(0, 2, 3, 1, 4).reshape(bsz, hkv, rep * lq, d)
        m = mask[:, None, None].expand(bsz, 1, rep, lq, mask.shape[-1]).reshape(bsz, 1, rep * lq, -1)
        o = self._sdpa(qg, kk, vv, m)
        return o.view(bsz, hkv, rep, lq, d).permute(0, 3, 1, 2, 4).reshape(bsz, lq, hkv * rep, d)

    @staticmethod
    def _key_slots(t, tables, lens, lmax, dev):
        """Slots of keys 0..lmax-1 through the page tables (clamped to a valid
        slot past each length; those keys are masked)."""
        j = t.arange(lmax, device=dev)
        jc = t.minimum(j[None, :], (lens[:, None] - 1).clamp(min=0))
        pages = tables.long().gather(1, jc // 256).clamp(min=0)
        return pages * 256 + jc % 256

    def decode(self, attn, x, positions, context_lens, block_tables, slot_mapping=None):
        t = self.torch
        q, k, v = self._project(attn, x, positions)
        self._store(attn, k, v, slot_mapping)
        key = ("d", id(context_lens))
        if self._meta_key != key:
            lens = context_lens.long() + 1
            lmax = int(lens.max())
            slots = self._key_slots(t, block_tables, lens, lmax, x.device)
            mask = t.arange(lmax, device=x.device)[None, :] < lens[:, None]
            self._meta_key, self._meta = key, (context_lens, slots, mask[:, None, :])
        _, slots, mask = self._meta
        o = self._attend(attn, q[:, None], slots, mask, 1)
        return attn.o_proj(o.reshape(x.shape[0], -1))

    def prefill(self, attn, x, positions, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                block_mapping, block_tables=None):
        t = self.torch
        q, k, v = self._project(attn, x, positions)
        self._store(attn, k, v, block_mapping)
        dev = x.device
        key = ("p", id(cu_seqlens_q))
        if self._meta_key != key:
            cq, ck = cu_seqlens_q.tolist(), cu_seqlens_k.tolist()
            lq = [cq[b + 1] - cq[b] for b in range(len(cq) - 1)]
            lk = [ck[b + 1] - ck[b] for b in range(len(ck) - 1)]
            groups = []
            for rows in ([b for b in range(len(lq)) if lq[b] == 1],
                         [b for b in range(len(lq)) if lq[b] > 1]):
                if not rows:
                    continue
                LQ = max(lq[b] for b in rows)
                LK = max(lk[b] for b in rows)
                rows_t = t.tensor(rows, device=dev)
                lq_t = t.tensor([lq[b] for b in rows], device=dev)
                lk_t = t.tensor([lk[b] for b in rows], device=dev)
                qi = t.tensor([cq[b] for b in rows], device=dev)[:, None] + t.arange(LQ, device=dev)[None]
                qvalid = t.arange(LQ, device=dev)[None] < lq_t[:, None]
                qi = t.where(qvalid, qi, t.zeros_like(qi))
                slots = self._key_slots(t, block_tables[rows_t], lk_t, LK, dev)
                i = t.arange(LQ, device=dev)[None, :, None]
                j = t.arange(LK, device=dev)[None, None, :]
                # bottom-right causal; padded query rows see key 0 only (discarded)
                mask = (j <= i + (lk_t - lq_t)[:, None, None]) & (j < lk_t[:, None, None])
                mask = mask | (~qvalid[:, :, None] & (j == 0))
                groups.append((LQ, qi, qvalid, slots, mask))
            self._meta_key, self._meta = key, (cu_seqlens_q, groups)
        _, groups = self._meta
        out = t.empty_like(q)
        for LQ, qi, qvalid, slots, mask in groups:
            o = self._attend(attn, q[qi], slots, mask, LQ)
            out[qi[qvalid]] = o[qvalid]
        return attn.o_proj(out.reshape(x.shape[0], -1))

    def __enter__(self):
        QN, me = self.QN, self
        self._saved = (QN._use_kernels, QN.Qwen3Attention.forward_decode,
                       QN.Qwen3Attention.forward_prefill)
        QN._use_kernels = lambda *a: False
        QN.Qwen3Attention.forward_decode = lambda attn, *a, **k: me.decode(attn, *a, **k)
        QN.Qwen3Attention.forward_prefill = lambda attn, *a, **k: me.prefill(attn, *a, **k)
        return self

    def __exit__(self, *exc):
        QN = self.QN
        QN._use_kernels, QN.Qwen3Attention.forward_decode, QN.Qwen3Attention.forward_prefill = self._saved
        return False


class ReferenceEngine:
    """The reference's rollout loop, generate_continuous_with_logprobs
    (qwen3_naive.py:1474-1679), restated over this model as the end-to-end
    baseline.  Kept from the reference:
      * the scheduler: decode first, LIFO preemption, 2,048-token budget
        (:1499-1585; the model's own _schedule, which follows it);
      * decode as HIP graphs only for batches of at most 64 (buckets
        1, 2, 4, 8, 16, 32, 48, 64, page-table width min(pool, 160),
        :1070-1145), eager above;
      * lm_head over every token of the step (:1607), then the sampled rows;
      * sampling with torch ops: fp32 logits / T, optional top-k mask,
        softmax, multinomial, log_softmax + gather (:1632-1650), and two
        .item() reads per sampled sequence (:1656-1659);
      * no decode lookahead.
    ``body``: "torch" runs TorchBody (eager at every batch size: a torch
    attention over varying lengths cannot be captured); "kernels" keeps this
    build's HIP kernels as stand-ins for the reference's flash-attn / Triton /
    inductor kernels (one fused kernel each there too), so only the engine
    structure differs from the product.  Bench-only."""

    GRAPH_BS = (1, 2, 4, 8, 16, 32, 48, 64)

    def __init__(self, torch, pkg, model, body):
        self.torch, self.pkg, self.m, self.body = torch, pkg, model, body
        self.stats = {}

    def _swap_graph_state(self, state=None):
        m = self.m
        keys = ("_graphs", "_graphs_units", "_graph_bufs", "_graph_pool", "_graph_in",
                "_graph_max_bs", "_has_cuda_graphs")
        old = {k: getattr(m, k, None) for k in keys}
        if state is not None:
            for k, v in state.items():
                setattr(m, k, v)
        return old

    def setup(self):
        """Capture the reference's decode graphs (kernels body), outside any timing."""
        if self.body != "kernels":
            return
        m = self.m
        saved = self._swap_graph_state()
        with self.torch.no_grad():
            m._init_cuda_graphs(max_bs=64, bt_width=min(m._num_blocks, 160))
            m._capture_decode_graphs(batch_sizes=self.GRAPH_BS)
        self._ref_state = self._swap_graph_state(saved)

    def generate(self, prompts, max_new_tokens, temperature=1.0, top_k=None):
        t, m, P = self.torch, self.m, self.pkg.paged
        from collections import deque
        bm = P.BlockManager(m._num_blocks, m.BLOCK_SIZE)
        waiting = deque(P.Sequence(p[0].tolist(), {"temperature": temperature,
                                                   "max_tokens": max_new_tokens})
                        for p in prompts)
        all_seqs = list(waiting)
        running = []
        m._preemptions = 0
        st = {"steps": 0, "decode_steps": 0, "graph_steps": 0, "item_reads": 0}
        ctx = TorchBody(t, self.pkg) if self.body == "torch" else None
        saved = self._swap_graph_state(getattr(self, "_ref_state", None)) if self.body == "kernels" else None
        try:
            if ctx is not None:
                ctx.__enter__()
            with t.no_grad():
                while waiting or running:
                    sched = m._schedule(waiting, running, bm)
                    if not sched:
                        continue
                    st["steps"] += 1
                    all_decode = all(s.num_scheduled_tokens == 1 for s in sched)
                    if all_decode:
                        st["decode_steps"] += 1
                        ids, pos, cl, bt, slots = m._prepare_decode(sched)
                        h = None
                        if self.body == "kernels" and len(sched) <= 64:
                            h = m._run_decode_graph(len(sched), ids, pos, cl, bt, slots)
                            st["graph_steps"] += h is not None
                        if h is None:
                            h = m.model.forward_decode(ids, pos, cl, bt, slots)
                    else:
                        ids, pos, cu_q, cu_k, mq, mk, bmap, bt = m._prepare_step(sched)
                        h = m.model.forward_prefill(ids, pos, cu_q, cu_k, mq, mk, bmap, bt)
                    logits = m.lm_head(h)
                    for s in sched:
                        s.kv_len += s.num_scheduled_tokens
                        if not all_decode:
                            bm.hash_blocks(s)
                    idx, off = [], 0
                    for s in sched:
                        if s.num_scheduled_tokens == 1 or s.kv_len >= s.num_prompt_tokens:
                            idx.append(off + s.num_scheduled_tokens - 1)
                        off += s.num_scheduled_tokens
                    if not idx:
                        for s in sched:
                            s.num_scheduled_tokens = 0
                        continue
                    last = logits[idx].float() / temperature
                    if top_k is not None:
                        vals, tix = t.topk(last, top_k, dim=-1)
                        last = t.full_like(last, float("-inf")).scatter(-1, tix, vals)
                    probs = t.softmax(last, dim=-1)
                    nxt = t.multinomial(probs, num_samples=1)
                    slp = t.log_softmax(last, dim=-1).gather(-1, nxt)
                    j = 0
                    for s in sched:
                        if s.num_scheduled_tokens == 1 or s.kv_len >= s.num_prompt_tokens:
                            tok = nxt[j].item()
                            s.append_token(tok)
                            s.response_log_probs.append(slp[j].item())
                            st["item_reads"] += 2
                            j += 1
                            if s.num_completion_tokens >= s.max_tokens:
                                s.status = "FINISHED"
                                bm.deallocate(s.block_table)
                                s.block_table.clear()
                                running.remove(s)
                        s.num_scheduled_tokens = 0
        finally:
            if ctx is not None:
                ctx.__exit__(None, None, None)
            if saved is not None:
                self._ref_state = self._swap_graph_state(saved)
        st["preemptions"] = m._preemptions
        self.stats = st
        return ([s.token_ids for s in all_seqs], [s.token_ids[s.num_prompt_tokens:] for s in all_seqs],
                [list(s.response_log_probs) for s in all_seqs], [s.num_prompt_tokens for s in all_seqs])


def make_rollout_model(torch, pkg, dev, pool_gb=40.0):
    """Random-init Qwen3-0.6B (28 layers, tied lm_head, transformers' N(0, 0.02)
    initialisation) in bf16 with a KV pool of ``pool_gb`` GB (40 GB -> 1,362
    blocks of 29.36 MB)."""
    model = make_qwen3(torch, pkg, dev)
    model.allocate_global_kv_cache(num_blocks=int(pool_gb * 1e9 // model.kv_block_bytes()))
    return model


def rollout_prompts(torch, n_prompts=32, group=8, prompt_len=128, vocab=151936, seed=0):
    g = torch.Generator().manual_seed(seed)
    base = [torch.randint(0, vocab, (1, prompt_len), generator=g) for _ in range(n_prompts)]
    return [p for p in base for _ in range(group)]


def grpo_loss_after_rollout(torch, pkg, model, seqs, plens, lps, n_prompts, group, micro=32, seed=0):
    """New log-probs of every generated token (prefill forward to the final
    hidden states, then the fused lm_head + log-prob kernel: no logits are
    materialised), seeded Bernoulli(0.5) rewards, group advantages and the
    clipped loss (per-sequence masked mean), next-token alignment;
    micro-batched over sequences (32 sequences = 36,864 rows per forward: the
    loss step took 0.567 / 0.537 / 0.540 s at 16 / 32 / 64)."""
    dev = next(model.parameters()).device
    g = torch.Generator().manual_seed(seed)
    rewards = torch.bernoulli(torch.full((len(seqs),), 0.5), generator=g).to(dev)
    pids = torch.arange(n_prompts).repeat_interleave(group).to(dev)
    total, n_seq = 0.0, len(seqs)
    with torch.no_grad():
        for s0 in range(0, n_seq, micro):
            chunk = seqs[s0:s0 + micro]
            T = max(len(x) for x in chunk)
            bm = pkg.BlockManager(model._num_blocks)
            objs = []
            for toks in chunk:
                sq = pkg.Sequence(toks)
                bm.allocate(sq)
                sq.kv_len = 0
                sq.num_scheduled_tokens = len(toks)
                objs.append(sq)
            ids, pos, cu_q, cu_k, mq, mk, bmap, bt = model._prepare_step(objs)
            h = model.model.forward_prefill(ids, pos, cu_q, cu_k, mq, mk, bmap, bt)
            ids2 = ids.view(len(chunk), T)
            old = torch.zeros((len(chunk), T), dtype=torch.float32, device=dev)
            mask = torch.zeros_like(old)
            for i, (pl, lp) in enumerate(zip(plens[s0:s0 + micro], lps[s0:s0 + micro])):
                old[i, pl:pl + len(lp)] = torch.tensor(lp, device=dev)
                mask[i, pl:pl + len(lp)] = 1.0
            loss, _, _ = pkg.grpo_loss_from_hidden(h.view(len(chunk), T, -1), model.lm_head.weight,
                                                   ids2, old, mask, rewards[s0:s0 + micro],
                                                   pids[s0:s0 + micro], 1e-4, 0.2, "seq",
                                                   shift=True)
            total += loss.item() * len(chunk) / n_seq
            del h
    return total


def _timed(torch, fn):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, time.perf_counter() - t0


def leg_rollout(torch, pkg, dev, new_tokens=1024, compare_tokens=64, preempt_blocks=1200,
                engines=("ours", "kernels", "torch"), runs_n=3, cpu=False, eos_runs=True):
    """Config 5: 32 prompts x group 8 = 256 sequences, 128-token prompts, T=1.0,
    no top-k, ``new_tokens`` generated tokens each, continuous batching with the
    2048-token step budget and LIFO preemption, ~40 GB pool (1,362 blocks: no
    preemption); then the GRPO loss over the generated tokens.  Also: the same
    rollout in a ``preempt_blocks`` pool (under the 1,280 blocks 256 x 5 pages
    need, so LIFO preemption fires), and ours against the reference engine's
    loop (ReferenceEngine, two model bodies) at ``compare_tokens`` new tokens, and
    (``eos_runs``) EOS-terminated rollouts in the ~40 GB pool."""
    model = make_rollout_model(torch, pkg, dev)
    prompts = rollout_prompts(torch)
    n_tok = len(prompts)
    gen = lambda n, **k: model.generate_continuous_with_logprobs(
        prompts, max_new_tokens=n, temperature=1.0, top_k=None, **k)
    log("rollout: warm-up / graph capture")
    model.generate_continuous_with_logprobs(prompts[:16], max_new_tokens=4, temperature=1.0,
                                            top_k=None)
    out = {}
    if compare_tokens > 0:
        if "ours" in engines:
            torch.manual_seed(1)
            _, dt = _timed(torch, lambda: gen(compare_tokens))
            out["ours_short"] = dict(tokens_per_s=n_tok * compare_tokens / dt, s=dt,
                                     **dict(model.last_stats))
            log(f"rollout: ours {out['ours_short']['tokens_per_s']:.0f} tok/s at "
                f"{compare_tokens} tokens")
        for body in [e for e in ("kernels", "torch") if e in engines]:
            ref = ReferenceEngine(torch, pkg, model, body)
            ref.setup()
            torch.manual_seed(1)
            _, dt = _timed(torch, lambda: ref.generate(prompts, compare_tokens, 1.0, None))
            out[f"reference_{body}_short"] = dict(tokens_per_s=n_tok * compare_tokens / dt, s=dt,
                                                  **ref.stats)
            log(f"rollout: reference engine ({body} body) "
                f"{out[f'reference_{body}_short']['tokens_per_s']:.0f} tok/s")
            del ref
        torch.cuda.empty_cache()
    if new_tokens <= 0:
        del model
        torch.cuda.empty_cache()
        return out
    # Three timed runs (rollout, then the loss over its tokens), median reported;
    # the short capture run above is the warm-up.
    runs = []
    for i in range(runs_n):
        log(f"rollout: full run {i + 1}/{runs_n} ({n_tok} x {new_tokens} tokens)")
        torch.manual_seed(2 + i)
        (toks, gen_t, lps, plens), t_roll = _timed(torch, lambda: gen(new_tokens))
        stats = dict(model.last_stats)
        t0 = time.perf_counter()
        loss = grpo_loss_after_rollout(torch, pkg, model, toks, plens, lps, 32, 8)
        torch.cuda.synchronize()
        t_loss = time.perf_counter() - t0
        generated = sum(len(x) for x in gen_t)
        assert len(set(len(x) for x in toks)) == 1, "fixed-length rollout expected (no EOS)"
        runs.append(dict(rollout_s=t_roll, loss_s=t_loss, loss=loss, stats=stats))
        del toks, gen_t, lps
    med = sorted(runs, key=lambda r: r["rollout_s"])[len(runs) // 2]
    t_roll, t_loss = med["rollout_s"], med["loss_s"]
    out.update(dict(generated=generated, rollout_s=t_roll, loss_s=t_loss, loss=med["loss"],
                    tokens_per_s=generated / t_roll,
                    tokens_per_s_with_loss=generated / (t_roll + t_loss),
                    runs_tokens_per_s=[generated / r["rollout_s"] for r in runs],
                    num_blocks=model._num_blocks, **med["stats"]))
    if preempt_blocks:
        log(f"rollout: {preempt_blocks}-block pool (forced LIFO preemption)")
        model.allocate_global_kv_cache(num_blocks=preempt_blocks)
        model.generate_continuous_with_logprobs(prompts[:16], max_new_tokens=4, temperature=1.0,
                                                top_k=None)
        torch.manual_seed(2)
        (_, gen_p, _, _), dt = _timed(torch, lambda: gen(new_tokens))
        gen_n = sum(len(x) for x in gen_p)
        assert gen_n == generated
        out["preempt"] = dict(num_blocks=preempt_blocks, rollout_s=dt, tokens_per_s=gen_n / dt,
                              **dict(model.last_stats))
        log(f"rollout: preemption run {gen_n / dt:.0f} tok/s, "
            f"{model.last_stats['preemptions']} preemptions")
        model.allocate_global_kv_cache(num_blocks=out["num_blocks"])
        model.generate_continuous_with_logprobs(prompts[:16], max_new_tokens=4, temperature=1.0,
                                                top_k=None)
    if eos_runs:
        # EOS-terminated rollouts: Qwen3's end ids (<|endoftext|>, <|im_end|>), and a
        # dense set (every 1,024th id: ~1e-3 per token on the random-init model, so
        # about 60% of the sequences stop early and the decode batch thins out).
        vocab = model.config.vocab_size
        for name, ids in (("eos", [151643, 151645]), ("eos_varlen", list(range(7, vocab, 1024)))):
            ids = [i for i in ids if i < vocab]
            torch.manual_seed(2)
            (_, gen_e, _, _), dt = _timed(torch, lambda: gen(new_tokens, eos_token_ids=ids))
            gen_n = sum(len(x) for x in gen_e)
            out[name] = dict(eos_ids=len(ids), generated=gen_n, rollout_s=dt,
                             tokens_per_s=gen_n / dt,
                             finished_early=sum(len(x) < new_tokens for x in gen_e),
                             mean_new_tokens=gen_n / len(gen_e), **dict(model.last_stats))
            log(f"rollout: {name} run {gen_n / dt:.0f} tok/s, "
                f"{out[name]['finished_early']} sequences ended at EOS")
    if cpu:
        log("cpu baseline (oracle decode steps at batch 256)")
        out["cpu_baseline"] = cpu_baseline_rollout(torch, model)
    del model
    torch.cuda.empty_cache()
    return out


def cpu_baseline_rollout(torch, model, steps=2, ctx=640, batch=256):
    """Config 5 on the host cores, sampled: ``steps`` decode steps of the
    oracle's 28-layer model (fp32 torch CPU, qwen3_decode_step) for ``batch``
    sequences at the rollout's mean context (every sequence with ``ctx``
    cached keys of random K/V, the same rows in every layer), the model's own
    random-init weights; tokens/s = batch x steps / time."""
    from oracle import model as OM
    torch.set_num_threads(os.cpu_count() or 1)
    cfg = model.config
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}  # fp32 once
    g = torch.Generator().manual_seed(5)
    k_rows = [torch.randn(ctx, cfg.num_key_value_heads, cfg.head_dim, generator=g)
              .to(torch.bfloat16) for _ in range(batch)]
    v_rows = [torch.randn(ctx, cfg.num_key_value_heads, cfg.head_dim, generator=g)
              .to(torch.bfloat16) for _ in range(batch)]
    k_ctx = [k_rows] * cfg.num_hidden_layers
    v_ctx = [v_rows] * cfg.num_hidden_layers
    tok = torch.randint(0, cfg.vocab_size, (batch,), generator=g)
    pos = torch.full((batch,), ctx, dtype=torch.int64)
    times = []
    for _ in range(steps):
        t = time.perf_counter()
        OM.qwen3_decode_step(sd, tok, pos, k_ctx, v_ctx, cfg.num_hidden_layers,
                             cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                             cfg.rms_norm_eps, cfg.rope_theta)
        times.append(time.perf_counter() - t)
    dt = statistics.median(times)
    return dict(value=batch / dt, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"oracle 28-layer decode step (fp32 torch CPU) for {batch} sequences with "
                       f"{ctx} cached keys each (the rollout's mean context), median of {steps} "
                       f"steps",
                seconds_per_sample=dt, cpu_model=_cpu_model())


def leg_copy_calibration(torch, dev, nbytes=1 << 30):
    """A plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE."""
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return dict(bytes_read=nbytes, bytes_written=nbytes)


# ---------------------------------------------------------------------------
def leg_decode_small(torch, pkg, W, dev, steps=200, warmup=20):
    """Config 1: one attention layer's decode step for 4 sequences (contexts
    37/256/300/700): store the new K/V, then paged decode over 1,297 keys
    (5,312,512 B of K/V, cache-resident).  Reported in µs per step, beside the
    oracle's fp32 CPU step on the host cores."""
    from oracle import attention as OA
    from oracle import paged as OP
    w = W.decode_one_layer(seed=0)
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in w.items()}
    out = torch.empty_like(g["q"])

    def step():
        pkg.kernels.store_kvcache(g["k_new"], g["v_new"], g["k_cache"], g["v_cache"],
                                  g["slot_mapping"])
        pkg.kernels.paged_decode_attention(g["q"], g["k_cache"], g["v_cache"],
                                           g["context_lens"], g["block_tables"], g["scale"],
                                           seqlen_bias=1, out=out)
    # Captured as a HIP graph of `per_graph` consecutive steps and replayed:
    # a step's launches take less GPU time than the host-side argument checks
    # of its calls, or than one graph launch.
    per_graph = 20
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            step()
    n_rep = max(1, steps // per_graph)
    total_ms, _ = timed_launches(torch, [graph.replay], n_rep, max(1, warmup // per_graph))
    total_ms *= steps / (n_rep * per_graph)
    eager_ms, _ = timed_launches(torch, [step], max(10, steps // 10), 2)
    k_ref, v_ref = w["k_cache"].clone(), w["v_cache"].clone()

    def cpu_step():
        OP.store_kvcache(w["k_new"], w["v_new"], k_ref, v_ref, w["slot_mapping"])
        return OA.paged_decode(w["q"], k_ref, v_ref, w["cache_seqlens"], w["block_tables"],
                               w["scale"])
    torch.set_num_threads(os.cpu_count() or 1)
    times = []
    for _ in range(4):
        t = time.perf_counter()
        ref = cpu_step()
        times.append(time.perf_counter() - t)
    err = (out.float().cpu() - ref).abs().max().item()
    slots_exact = torch.equal(g["k_cache"].cpu(), k_ref) and torch.equal(g["v_cache"].cpu(), v_ref)
    return dict(us_per_step=total_ms / steps * 1e3,
                eager_us_per_step=eager_ms / max(10, steps // 10) * 1e3, max_abs_err_vs_oracle=err,
                kv_cache_bit_exact=slots_exact, kv_bytes=5312512, note="store + decode of one layer; 5.3 MB of K/V is "
                "cache-resident, so no HBM fraction is claimed",
                cpu_oracle_us=statistics.median(times[1:]) * 1e6,
                cpu_cores=torch.get_num_threads())


def cpu_baseline_decode(torch, W, wdec, budget_s=10.0):
    """The oracle's paged decode (fp32, torch CPU) over the 64 sequences of one
    layer, repeated for about ``budget_s`` seconds (bounded sample)."""
    from oracle import attention as OA
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q = wdec["q"].cpu()
    kc = wdec["k_cache"][0].cpu()
    vc = wdec["v_cache"][0].cpu()
    lens = wdec["cache_seqlens"].cpu()
    bt = wdec["block_tables"].cpu()
    scale = wdec["scale"]
    nbytes = W.decode_kv_bytes(lens)
    OA.paged_decode(q[:2], kc, vc, lens[:2], bt[:2], scale)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start) < budget_s:
        t = time.perf_counter()
        OA.paged_decode(q, kc, vc, lens, bt, scale)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return dict(value=nbytes / med / 1e9, unit="GB/s", cores=torch.get_num_threads(),
                kind="port",
                sample=f"oracle paged decode (fp32 torch CPU) over all 64 sequences of one layer "
                       f"({nbytes / 1e6:.1f} MB of K/V), median of {len(times)} runs "
                       f"(~{budget_s:.0f} s)",
                seconds_per_sample=med, cpu_model=_cpu_model())


def cpu_baseline_grpo(torch, budget_rows=512, budget_s=10.0):
    """The oracle's fp32 log-softmax gather + loss over 512 rows of the loss step,
    repeated for about ``budget_s`` seconds (median run)."""
    from oracle import grpo as OG
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(1, budget_rows, 151936, generator=g) * 2).to(torch.bfloat16)
    ids = torch.randint(0, 151936, (1, budget_rows), generator=g)
    mask = torch.ones(1, budget_rows)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start) < budget_s:
        t = time.perf_counter()
        lp, _ = OG.logprob_gather(logits, ids)
        OG.ppo_loss_and_grad(lp + 0.01, lp, torch.ones(1, budget_rows), mask, 0.2, "seq")
        times.append(time.perf_counter() - t)
    dt = statistics.median(times)
    return dict(value=budget_rows * 151936 * 2 / dt / 1e9, unit="GB/s",
                cores=torch.get_num_threads(), kind="port",
                sample=f"oracle fp32 log-softmax gather + clipped loss over {budget_rows} rows "
                       f"of vocab 151936, median of {len(times)} runs (~{budget_s:.0f} s)",
                seconds_per_sample=dt)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--legs",
                    default="decode1,decode,decode_step,decode_step256,lm_head,grpo,store,prefill,norm_rope,host,"
                            "rollout")
    ap.add_argument("--rollout-tokens", type=int, default=1024,
                    help="new tokens per sequence in the end-to-end rollout leg")
    ap.add_argument("--rollout-compare-tokens", type=int, default=64,
                    help="new tokens of the short ours-vs-reference-engine comparison (0 skips it)")
    ap.add_argument("--rollout-engines", default="ours,kernels,torch",
                    help="engines of that comparison: ours, kernels (reference loop, this "
                         "build's kernels), torch (reference loop, torch body)")
    ap.add_argument("--rollout-preempt-blocks", type=int, default=1200,
                    help="pool of the forced-preemption rollout (0 skips it)")
    ap.add_argument("--rollout-runs", type=int, default=3,
                    help="timed full rollouts (median reported)")
    ap.add_argument("--rollout-no-eos", action="store_true",
                    help="skip the EOS-terminated rollout runs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device copy (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build targets a single MI355X and has no "
              "multi-GPU path (run with --gpus 1).", file=sys.stderr)
        return 2

    import torch
    from oracle import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (none visible)", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        print(json.dumps(leg_copy_calibration(torch, dev)))
        return 0
    pkg = load_pkg()
    legs = set(args.legs.split(","))

    torch.cuda.synchronize()
    results = {}
    cpu = None
    if "decode1" in legs:
        results["decode1"] = leg_decode_small(torch, pkg, W, dev)
    if "decode" in legs:
        results["decode"] = leg_decode(torch, pkg, W, dev, args.steps, args.warmup)
        if not args.no_cpu:
            log("cpu baseline (oracle decode)")
            cpu = cpu_baseline_decode(torch, W, results["decode"]["workload"])
        results["decode"]["kv_pool_gb"] = results["decode"]["workload"]["k_cache"].numel() * 4 / 1e9
        if "decode_step" in legs:
            results["decode_step"] = leg_decode_step(torch, pkg, dev, max(5, args.steps // 2),
                                                     args.warmup, results["decode"]["workload"],
                                                     results["decode"]["ms_per_step"])
        del results["decode"]["workload"]
        torch.cuda.empty_cache()
    if "decode_step256" in legs:
        results["decode_step256"] = leg_decode_step256(torch, pkg, dev, max(5, args.steps // 2),
                                                       args.warmup)
    if "lm_head" in legs:
        results["lm_head"] = leg_lm_head(torch, pkg, dev, args.steps, args.warmup)
    if "grpo" in legs:
        results["grpo"] = leg_grpo(torch, pkg, W, dev, max(3, args.steps // 2), args.warmup)
    if "store" in legs:
        results["store"] = leg_store(torch, pkg, dev, args.steps, args.warmup, cpu=not args.no_cpu)
    if "prefill" in legs:
        results["prefill"] = leg_prefill(torch, pkg, W, dev, max(3, args.steps // 2), args.warmup,
                                         cpu=not args.no_cpu)
    if "norm_rope" in legs:
        results["norm_rope"] = leg_norm_rope(torch, pkg, dev, args.steps, args.warmup)
    if "host" in legs:
        results["host"] = leg_host_prepare(torch, pkg)
    if "rollout" in legs:
        results["rollout"] = leg_rollout(torch, pkg, dev, new_tokens=args.rollout_tokens,
                                         compare_tokens=args.rollout_compare_tokens,
                                         preempt_blocks=args.rollout_preempt_blocks,
                                         engines=tuple(args.rollout_engines.split(",")),
                                         runs_n=args.rollout_runs, cpu=not args.no_cpu,
                                         eos_runs=not args.rollout_no_eos)

    cpu_grpo = None
    if not args.no_cpu and "grpo" in results:
        log("cpu baseline (oracle grpo)")
        cpu_grpo = cpu_baseline_grpo(torch)

    secondary = {}
    if "grpo" in results:
        r = results["grpo"]
        secondary["grpo_logprob_loss"] = {
            "workload": "fused log-softmax gather + group advantages + clipped loss, "
                        "32x512 rows, vocab 151936, bf16 logits, fp32 math",
            "us_per_launch": round(r["avg_launch_us"], 2), "gbs": round(r["gbs"], 1),
            "frac_of_hbm_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": r["bytes_per_launch"], "loss": r["loss"],
            "cpu_baseline": cpu_grpo}
        secondary["grpo_logprob_backward"] = {
            "workload": "d loss / d logits through log_softmax (bf16 out), same 32x512x151936 "
                        "rows; masked rows only write zeros",
            "us_per_launch": round(r["bwd_avg_launch_us"], 2), "gbs": round(r["bwd_gbs"], 1),
            "frac_of_hbm_peak": round(r["bwd_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": r["bwd_bytes_per_launch"], "active_rows": r["bwd_active_rows"]}
    if "store" in results:
        r = results["store"]
        secondary["kv_store"] = {
            "workload": f"slot-mapped KV store, {r['tokens']} tokens x 2 x 1024 bf16",
            "us_per_launch": round(r["avg_launch_us"], 2), "gbs": round(r["gbs"], 1),
            "frac_of_hbm_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": r["bytes_per_launch"]}
        secondary["kv_store"]["workload"] += (f", {r['rotating_sets']} rotating input/pool sets "
                                              "(no reuse through the Infinity Cache)")
        for k in ("rows_bit_exact_vs_oracle", "cpu_baseline"):
            if k in r:
                secondary["kv_store"][k] = r[k]

    if "norm_rope" in results:
        secondary["qk_norm_rope_store"] = {
            "workload": "fused per-head QK-RMSNorm + RoPE + KV store, Hq 16 / Hkv 8, head_dim 128 "
                        "(16,908 B per token: qkv row, position, slot and cos/sin row in; q, "
                        "K and V rows out); RMSNorm / add + RMSNorm / SwiGLU over 8,192 rows; "
                        "HIP graphs of 20 launches", **results["norm_rope"]}

    if "lm_head" in results:
        secondary["lm_head_fused"] = {
            "workload": "fused lm_head (hidden 1024 x vocab 151936 bf16, fp32 logits never "
                        "materialised) + inverse-CDF sampling with the drawn token's log-prob "
                        "(sample_*), or + target log-prob gather (logprob_*); against the "
                        "unfused hipBLASLt GEMM + streaming sampler / log-prob kernel",
            **results["lm_head"]}

    if "decode_step" in results:
        r = results["decode_step"]
        secondary["decode_step_28layer_b64"] = {
            "workload": "one full Qwen3-0.6B decode step (28 layers, random-init bf16 weights) "
                        "for 64 sequences, contexts U{1024..4096}, shuffled page tables, as the "
                        "engine's HIP graph (embedding, norms, GEMMs, paged attention with the "
                        "QK-norm/RoPE/KV store folded in, SwiGLU, final norm); the fused lm_head + sampler "
                        "(logits never materialised) timed after it; the unfused [64, V] lm_head "
                        "GEMM alone for comparison",
            "ms_per_step": round(r["ms_per_step"], 4),
            "ms_per_step_with_lm_head_and_sampling":
                round(r["ms_per_step_with_lm_head_and_sampling"], 4),
            "unfused_lm_head_gemm_ms": round(r["unfused_lm_head_gemm_ms"], 4),
            "attention_ms_per_step": round(r["attention_ms_per_step"], 4),
            "attention_share": round(r["attention_share"], 4),
            "kv_bytes_per_step": r["kv_bytes_per_step"], "weight_bytes": r["weight_bytes"],
            "hbm_gbs_kv_plus_weights": round(r["hbm_gbs"], 1),
            "frac_of_hbm_peak": round(r["hbm_gbs"] / HBM_PEAK_GBS, 4)}

    if "decode_step256" in results:
        r = results["decode_step256"]
        secondary["decode_step_28layer_b256_rollout_shape"] = {
            "workload": "the rollout's decode step: 256 sequences x 640 cached keys (its mean "
                        "context), random-init Qwen3-0.6B bf16, 28 per-layer page pools, through "
                        "the engine's decode path (one input copy, then the whole-unit HIP graph "
                        "of the 256-row bucket); then the fused lm_head + sampler, all entries "
                        "and top 20",
            **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()},
            "frac_of_hbm_peak": round(r["hbm_gbs"] / HBM_PEAK_GBS, 4)}

    if "host" in results:
        secondary["host_decode_prepare"] = {
            "workload": "host-side decode step inputs (new-token slots, -1-padded page tables, "
                        "ids, positions, context lengths) for 256 sequences", **results["host"]}

    if "decode1" in results:
        r = results["decode1"]
        secondary["decode_one_layer_4seq"] = {
            "workload": "one layer's decode step, 4 sequences, contexts 37/256/300/700 "
                        "(store + paged decode over 1,297 keys), HIP graph of 20 steps",
            "us_per_step": round(r["us_per_step"], 2),
            "us_per_step_eager_calls": round(r["eager_us_per_step"], 2),
            "max_abs_err_vs_oracle": r["max_abs_err_vs_oracle"],
            "kv_cache_bit_exact": r["kv_cache_bit_exact"], "note": r["note"],
            "cpu_oracle_us": round(r["cpu_oracle_us"], 1), "cpu_cores": r["cpu_cores"]}

    if "prefill" in results:
        r = results["prefill"]
        secondary["prefill_attention"] = {
            "workload": "varlen paged causal prefill, 16 seqs sharing a cached 512-token prefix, "
                        "suffixes U{256..2048} in 512-token chunks, one layer (all chunk steps)",
            "ms_per_layer": round(r["ms_per_layer"], 4), "tflops": round(r["tflops"], 1),
            "frac_of_bf16_mfma_peak": round(r["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
            "flops_per_layer": r["flops"], "causal_pairs": r["causal_pairs"],
            "chunk_steps": r["n_steps"], "query_tokens": r["q_tokens"],
            "ms_per_layer_sum_of_launch_events": round(r["ms_per_layer_launch_events"], 4)}
        for k in ("max_abs_err_vs_oracle", "cpu_baseline"):
            if k in r:
                secondary["prefill_attention"][k] = r[k]

    if "rollout" in results and "tokens_per_s" in results["rollout"]:
        r = results["rollout"]
        secondary["grpo_rollout"] = {
            "workload": "random-init Qwen3-0.6B bf16, 32 prompts x group 8 = 256 seqs, 128-token "
                        f"prompts, {args.rollout_tokens} new tokens, T=1.0, no top-k, continuous "
                        "batching (2048-token budget, LIFO preemption), ~40 GB KV pool, then "
                        "per-token logprob gather + group advantages + clipped loss",
            "tokens_per_s": round(r["tokens_per_s"], 1),
            "tokens_per_s_with_loss": round(r["tokens_per_s_with_loss"], 1),
            "generated_tokens": r["generated"], "rollout_s": round(r["rollout_s"], 3),
            "loss_s": round(r["loss_s"], 3), "loss": r["loss"], "kv_blocks": r["num_blocks"],
            "preemptions": r.get("preemptions"), "engine_steps": r.get("steps"),
            "graph_decode_steps": r.get("graph_steps"),
            "lookahead_decode_steps": r.get("lookahead_steps"),
            "runs": len(r["runs_tokens_per_s"]),
            "runs_tokens_per_s": [round(x, 1) for x in r["runs_tokens_per_s"]],
            "cpu_baseline": r.get("cpu_baseline")}
        if "preempt" in r:
            pr = r["preempt"]
            secondary["grpo_rollout"]["forced_preemption"] = {
                "kv_blocks": pr["num_blocks"], "tokens_per_s": round(pr["tokens_per_s"], 1),
                "rollout_s": round(pr["rollout_s"], 3), "preemptions": pr["preemptions"],
                "engine_steps": pr["steps"], "graph_decode_steps": pr["graph_steps"],
                "lookahead_decode_steps": pr["lookahead_steps"]}
        for name, desc in (("eos", "Qwen3's end ids 151643 / 151645"),
                           ("eos_varlen", "every 1,024th vocabulary id (lengths vary)")):
            if name in r:
                e = r[name]
                secondary["grpo_rollout"][f"{name}_terminated"] = {
                    "eos_token_ids": desc, "tokens_per_s": round(e["tokens_per_s"], 1),
                    "generated_tokens": e["generated"], "rollout_s": round(e["rollout_s"], 3),
                    "finished_early": e["finished_early"],
                    "mean_new_tokens": round(e["mean_new_tokens"], 1),
                    "engine_steps": e["steps"], "graph_decode_steps": e["graph_steps"],
                    "lookahead_decode_steps": e["lookahead_steps"],
                    "discarded_rows": e.get("discarded_rows")}
        if "ours_short" in r:
            o = r["ours_short"]
            cmp = {"new_tokens": args.rollout_compare_tokens,
                   "ours_tokens_per_s": round(o["tokens_per_s"], 1)}
            for body, desc in (
                    ("kernels", "the reference's engine loop (graphs only up to batch 64, "
                                "lm_head over every token, torch softmax / multinomial / "
                                "log_softmax with two .item() per sequence per step, no "
                                "lookahead) with this build's kernels standing in for its "
                                "flash-attn / Triton / inductor kernels"),
                    ("torch", "the same loop with a torch body: torch norms / RoPE / SwiGLU / "
                              f"store and {TorchBody.attention_kind} over the K/V each "
                              "sequence needs, eager at every batch size (flash-attn is not "
                              "installed)")):
                rr = r.get(f"reference_{body}_short")
                if rr is None:
                    continue
                cmp[f"reference_engine_{body}_body"] = {
                    "description": desc, "tokens_per_s": round(rr["tokens_per_s"], 1),
                    "engine_steps": rr["steps"], "decode_steps": rr["decode_steps"],
                    "graph_decode_steps": rr["graph_steps"],
                    "ms_per_step": round(rr["s"] / rr["steps"] * 1e3, 3),
                    "speedup_of_ours": round(o["tokens_per_s"] / rr["tokens_per_s"], 2)}
            cmp["ours_ms_per_step"] = round(o["s"] / o["steps"] * 1e3, 3)
            secondary["grpo_rollout"]["reference_engine_comparison"] = cmp

    if "decode" in results:
        d = results["decode"]
        line = {
            "metric": METRIC,
            "value": round(d["gbs"], 1),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(d["ms_per_step"], 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) bf16 K/V pools and queries, shuffled block tables)",
            "config": {
                "workload": "paged GQA decode attention, one 28-layer Qwen3-0.6B decode step",
                "batch": 64, "context": "U{1024..4096}", "mean_context": round(d["mean_ctx"], 1),
                "q_heads": 16, "kv_heads": 8, "head_dim": 128, "page_tokens": 256,
                "layers": d["layers"],
                "kv_pool_gb": round(d["kv_pool_gb"], 2),
                "timing": "28 launches captured in one HIP graph, replayed back to back "
                          "(events around the replays)",
                "ms_per_step_eager_calls": round(d["eager_ms_per_step"], 4)},
            "roofline": {
                "bound": "hbm", "achieved": round(d["launch_gbs"], 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(d["launch_gbs"] / HBM_PEAK_GBS, 4),
                "traffic": DECODE_TRAFFIC_BYTES,
                "traffic_note": "HBM bytes per launch (split + merge) from rocprofv3 FETCH_SIZE x2.0 "
                                "+ WRITE_SIZE x1.0 passes of this leg, "
                                "profiles/paged_decode_28layer_b64_ctx1024-4096.md",
                "kernel": "decode_streamk_split<8, 2, 8, false> (+ decode_streamk_merge<8, 2, 8>)",
                "us_per_launch": round(d["avg_launch_us"], 2),
                "bytes_per_launch": d["bytes_per_launch"]},
            "cpu_baseline": cpu,
            "secondary": secondary,
        }
    else:
        line = {"metric": METRIC, "value": None, "secondary": secondary}
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
