#!/usr/bin/env python3
"""Benchmark of the GRPO rollout-and-loss hot path on one MI355X.

Headline (``value``): paged decode attention HBM GB/s for one full decode
step of Qwen3-0.6B at the serving shape -- 28 layers, 64 sequences with
contexts ~ U{1024..4096}, 16 query / 8 KV heads, head_dim 128, 256-token
pages with shuffled block tables.  Each layer owns its own K/V pool (18.8 GB
in total), so the 256 MB Infinity Cache cannot serve the reads.  A "step" is
the 28 decode-attention launches of one decode step.

Secondary legs (same JSON line): the fused GRPO logprob+advantage+loss kernel
on the 32x512x151936 loss step, the KV store at 65,536 tokens, the varlen
paged prefill on the prefix-cache chunk workload (MFMA TFLOP/s), and the CPU
oracle (the CPU restatement of the reference semantics) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--legs decode,grpo,store,prefill]
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
METRIC = "decode-attn HBM GB/s (% of 8 TB/s); GRPO rollout tokens/s on 1 GPU"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_pkg():
    lib = ROOT / "qwen3-naive-inference_amd" / "libqwen3mi.so"
    if not lib.exists():
        importlib.import_module("__graft_entry__").build()
    return importlib.import_module("qwen3-naive-inference_amd")


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
    ms_step = total_ms / steps
    avg_launch_ms = statistics.mean(per)
    gbs_step = per_launch_bytes * layers / (ms_step * 1e-3) / 1e9
    gbs_launch = per_launch_bytes / (avg_launch_ms * 1e-3) / 1e9
    return dict(ms_per_step=ms_step, gbs=gbs_step, avg_launch_us=avg_launch_ms * 1e3,
                launch_gbs=gbs_launch, bytes_per_launch=per_launch_bytes,
                kv_bytes_per_launch=kv_bytes, layers=layers,
                mean_ctx=float(lens.float().mean().item() - 1),
                workload=w)


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
    del w, args, res
    torch.cuda.empty_cache()
    return out


def leg_store(torch, pkg, dev, steps, warmup, n_tok=65536):
    log(f"store: {n_tok} tokens")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    nb = n_tok // 256 + 16
    key = torch.randn((n_tok, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    val = torch.randn((n_tok, 8, 128), generator=g, device=dev).to(torch.bfloat16)
    kc = torch.empty((nb, 256, 8, 128), dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    gc = torch.Generator().manual_seed(0)
    slots = torch.randperm(nb * 256, generator=gc)[:n_tok].to(torch.int32).to(dev)
    fn = lambda: pkg.kernels.store_kvcache(key, val, kc, vc, slots)
    total_ms, per = timed_launches(torch, [fn], steps, warmup)
    nbytes = 2 * 2 * key.numel() * 2 + slots.numel() * 4
    ms = statistics.mean(per)
    return dict(avg_launch_us=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, bytes_per_launch=nbytes,
                tokens=n_tok)


def leg_prefill(torch, pkg, W, dev, steps, warmup):
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
    total_ms, per = timed_launches(torch, fns, steps, warmup)
    ms = total_ms / steps
    return dict(ms_per_layer=ms, tflops=flops / (ms * 1e-3) / 1e12, flops=flops,
                causal_pairs=pairs, n_steps=len(calls),
                q_tokens=sum(int(c["cu_seqlens_q"][-1]) for c in calls))


def leg_copy_calibration(torch, dev, nbytes=1 << 30):
    """A plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE."""
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return dict(bytes_read=nbytes, bytes_written=nbytes)


# ---------------------------------------------------------------------------
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
    while len(times) < 3 and (time.perf_counter() - t_start) < budget_s:
        t = time.perf_counter()
        OA.paged_decode(q, kc, vc, lens, bt, scale)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return dict(value=nbytes / med / 1e9, unit="GB/s", cores=torch.get_num_threads(),
                kind="port",
                sample=f"oracle paged decode (fp32 torch CPU) over all 64 sequences of one layer "
                       f"({nbytes / 1e6:.1f} MB of K/V), median of {len(times)} runs",
                seconds_per_sample=med, cpu_model=_cpu_model())


def cpu_baseline_grpo(torch, budget_rows=512):
    """The oracle's fp32 log-softmax gather + loss over 512 rows of the loss step."""
    from oracle import grpo as OG
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(1, budget_rows, 151936, generator=g) * 2).to(torch.bfloat16)
    ids = torch.randint(0, 151936, (1, budget_rows), generator=g)
    mask = torch.ones(1, budget_rows)
    t = time.perf_counter()
    lp, _ = OG.logprob_gather(logits, ids)
    OG.ppo_loss_and_grad(lp + 0.01, lp, torch.ones(1, budget_rows), mask, 0.2, "seq")
    dt = time.perf_counter() - t
    return dict(value=budget_rows * 151936 * 2 / dt / 1e9, unit="GB/s",
                cores=torch.get_num_threads(), kind="port",
                sample=f"oracle fp32 log-softmax gather + clipped loss over {budget_rows} rows "
                       "of vocab 151936")


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
    ap.add_argument("--legs", default="decode,grpo,store,prefill")
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
    if "decode" in legs:
        results["decode"] = leg_decode(torch, pkg, W, dev, args.steps, args.warmup)
    if "grpo" in legs:
        results["grpo"] = leg_grpo(torch, pkg, W, dev, max(3, args.steps // 2), args.warmup)
    if "store" in legs:
        results["store"] = leg_store(torch, pkg, dev, args.steps, args.warmup)
    if "prefill" in legs:
        results["prefill"] = leg_prefill(torch, pkg, W, dev, max(3, args.steps // 2), args.warmup)

    cpu = None
    if not args.no_cpu and "decode" in results:
        log("cpu baseline (oracle decode)")
        cpu = cpu_baseline_decode(torch, W, results["decode"]["workload"])
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
    if "store" in results:
        r = results["store"]
        secondary["kv_store"] = {
            "workload": f"slot-mapped KV store, {r['tokens']} tokens x 2 x 1024 bf16",
            "us_per_launch": round(r["avg_launch_us"], 2), "gbs": round(r["gbs"], 1),
            "frac_of_hbm_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": r["bytes_per_launch"]}

    if "prefill" in results:
        r = results["prefill"]
        secondary["prefill_attention"] = {
            "workload": "varlen paged causal prefill, 16 seqs sharing a cached 512-token prefix, "
                        "suffixes U{256..2048} in 512-token chunks, one layer (all chunk steps)",
            "ms_per_layer": round(r["ms_per_layer"], 4), "tflops": round(r["tflops"], 1),
            "frac_of_bf16_mfma_peak": round(r["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
            "flops_per_layer": r["flops"], "causal_pairs": r["causal_pairs"],
            "chunk_steps": r["n_steps"], "query_tokens": r["q_tokens"]}

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
                "kv_pool_gb": round(d["workload"]["k_cache"].numel() * 2 * 2 / 1e9, 2)},
            "roofline": {
                "bound": "hbm", "achieved": round(d["launch_gbs"], 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(d["launch_gbs"] / HBM_PEAK_GBS, 4),
                "traffic": None,
                "kernel": "paged_decode_split (+ paged_decode_merge)",
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
