"""The HIP kernels against the committed golden fixtures (tests/golden).

Tolerances: KV store and slots bit-exact; attention max abs 2e-2 (bf16 output);
log-probabilities, advantages and loss 1e-4 relative (|err| / max(|ref|, 1))."""
import pytest
import torch

import golden_io as G
from oracle import workloads as W

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs() / b.abs().clamp_min(1.0)).max().item()


def test_config1_store_and_decode(pkg, gpu):
    meta = G.load_json("config1_checksums.json")
    w = W.decode_one_layer(seed=meta["seed"])
    assert G.sha(w["k_cache"]) == meta["sha256"]["k_cache"]
    print("[golden] config1", flush=True)
    kc, vc = w["k_cache"].to(gpu), w["v_cache"].to(gpu)
    pkg.kernels.store_kvcache(w["k_new"].to(gpu), w["v_new"].to(gpu), kc, vc,
                              w["slot_mapping"].to(gpu))
    out = pkg.kernels.paged_decode_attention(w["q"].to(gpu), kc, vc, w["context_lens"].to(gpu),
                                             w["block_tables"].to(gpu), SCALE, seqlen_bias=1)
    torch.cuda.synchronize()
    assert G.sha(kc) == meta["sha256"]["k_cache_after_store"]
    assert G.sha(vc) == meta["sha256"]["v_cache_after_store"]
    ref = G.load("config1_out.safetensors")["out_fp32"]
    assert (out.float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("pps", [0, 1])
def test_decode_small(pkg, gpu, pps):
    f = G.load("decode_small.safetensors")
    kc, vc = G.decode_small_pool(f)
    print(f"[golden] decode small pps={pps}", flush=True)
    out = pkg.kernels.paged_decode_attention(f["q"].to(gpu), kc.to(gpu), vc.to(gpu),
                                             f["cache_seqlens"].to(gpu),
                                             f["block_tables"].to(gpu), SCALE,
                                             pages_per_split=pps)
    torch.cuda.synchronize()
    assert (out.float().cpu() - f["out_fp32"]).abs().max().item() <= 2e-2
    assert (out.float().cpu() - f["out_bf16_eager"]).abs().max().item() <= 2e-2


def test_prefill_small(pkg, gpu):
    f = G.load("prefill_small.safetensors")
    kc, vc = G.prefill_small_pool(f)
    kc, vc, bt = kc.to(gpu), vc.to(gpu), f["block_tables"].to(gpu)
    print("[golden] prefill small", flush=True)
    for step, lk in (("step1", 28), ("step2", 36)):
        out = pkg.kernels.varlen_prefill_attention(
            f[f"q_{step}"].to(gpu), kc, vc, f["cu_q"].to(gpu), f[f"cu_k_{step}"].to(gpu),
            8, lk, SCALE, True, bt)
        torch.cuda.synchronize()
        assert (out.float().cpu() - f[f"out_{step}_fp32"]).abs().max().item() <= 2e-2, step


@pytest.mark.parametrize("reduction", ["token", "seq"])
@pytest.mark.parametrize("eps", ["1e-8", "1e-4"])
def test_grpo_small(pkg, gpu, reduction, eps):
    f = G.load("grpo_small.safetensors")
    print(f"[golden] grpo small {reduction} eps={eps}", flush=True)
    r = pkg.kernels.grpo_fused_forward(f["logits"].to(gpu), f["ids"].to(gpu),
                                       f["old_lp"].to(gpu), f["mask"].to(gpu),
                                       f["rewards"].to(gpu), f["prompt_ids"].to(gpu),
                                       float(eps), 0.2, reduction)
    torch.cuda.synchronize()
    assert _rel(r["lp"], f["lp"]) <= 1e-4
    assert _rel(r["lse"], f["lse"]) <= 1e-4
    assert _rel(r["adv"], f[f"adv_eps{eps}"]) <= 1e-4
    assert _rel(r["loss"].reshape(1), f[f"loss_{reduction}_eps{eps}"]) <= 1e-4
    assert (r["dlp"].cpu() - f[f"dlp_{reduction}_eps{eps}"]).abs().max().item() <= 1e-5
