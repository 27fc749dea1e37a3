"""Writes the golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_fixtures.py

Every fixture is seeded and produced by the oracle (``oracle/``) or, for the
page-allocator trace, by replaying a fixed script of operations whose
expected states are also asserted here from the allocation rules of
qwen3_naive.py:240-375 (free list popped from the end, freed pages appended,
a hashed page revived on a prefix hit).  The reference ships no fixtures or
stored tensors of its own, so these are the only golden vectors.

Files:
  config1_checksums.json   config 1 (one decode layer, 4 seqs, ctx 37/256/300/700):
                           seed + SHA-256 of every input, the slot mapping and the
                           post-store caches
  config1_out.safetensors  the fp32 oracle output of config 1 (q [4,16,128])
  decode_small.safetensors reduced decode case: 4 pages x 16 used tokens
  prefill_small.safetensors two sequences with cached prefixes, two 8-token chunks
  grpo_small.safetensors   4 x 16 tokens over a 1024-token vocabulary
  block_manager_trace.json allocator operations and the state after each
"""
from __future__ import annotations

import hashlib
import importlib
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import attention as OA  # noqa: E402
from oracle import grpo as OG  # noqa: E402
from oracle import paged as OP  # noqa: E402
from oracle import workloads as W  # noqa: E402

HQ, HKV, D, P = 16, 8, 128, 256


def sha(t: torch.Tensor) -> str:
    """SHA-256 of a tensor's raw bytes (bf16 viewed as int16)."""
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


# ---------------------------------------------------------------------------
def config1():
    w = W.decode_one_layer(seed=0)
    k_ref, v_ref = w["k_cache"].clone(), w["v_cache"].clone()
    OP.store_kvcache(w["k_new"], w["v_new"], k_ref, v_ref, w["slot_mapping"])
    out = OA.paged_decode(w["q"], k_ref, v_ref, w["cache_seqlens"], w["block_tables"], w["scale"])
    sums = {k: sha(w[k]) for k in ("q", "k_new", "v_new", "k_cache", "v_cache", "block_tables",
                                   "slot_mapping", "cache_seqlens")}
    sums["k_cache_after_store"] = sha(k_ref)
    sums["v_cache_after_store"] = sha(v_ref)
    meta = {"seed": 0, "ctx": [37, 256, 300, 700], "num_blocks": 16,
            "slot_mapping": w["slot_mapping"].tolist(), "block_tables": w["block_tables"].tolist(),
            "sha256": sums}
    with open(os.path.join(HERE, "config1_checksums.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    save_file({"out_fp32": out.contiguous()}, os.path.join(HERE, "config1_out.safetensors"))


# ---------------------------------------------------------------------------
def decode_small():
    """4 sequences, one page each (pages 3, 0, 2, 1 of a 4-page pool), contexts
    3 / 9 / 15 / 16 keys; only the first 16 token rows of each page are stored."""
    g = torch.Generator().manual_seed(101)
    lens = torch.tensor([3, 9, 15, 16], dtype=torch.int32)
    table = torch.tensor([[3], [0], [2], [1]], dtype=torch.int32)
    q = torch.randn(4, HQ, D, generator=g).to(torch.bfloat16)
    k_rows = torch.randn(4, 16, HKV, D, generator=g).to(torch.bfloat16)   # [page, token, h, d]
    v_rows = torch.randn(4, 16, HKV, D, generator=g).to(torch.bfloat16)
    kc = torch.zeros(4, P, HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[:, :16] = k_rows
    vc[:, :16] = v_rows
    out = OA.paged_decode(q, kc, vc, lens, table, D ** -0.5)
    out_bf = OA.paged_decode(q, kc, vc, lens, table, D ** -0.5, mode="bf16_eager")
    save_file({"q": q, "k_rows": k_rows, "v_rows": v_rows, "cache_seqlens": lens,
               "block_tables": table, "out_fp32": out.contiguous(),
               "out_bf16_eager": out_bf.contiguous()},
              os.path.join(HERE, "decode_small.safetensors"))


# ---------------------------------------------------------------------------
def prefill_small():
    """Two sequences with cached prefixes of 20 and 5 tokens, then two chunk
    steps of 8 new queries each (keys 28/13 after step 1, 36/21 after step 2).
    Sequence 0 lives in page 1, sequence 1 in page 0 (2-page pool)."""
    g = torch.Generator().manual_seed(202)
    total = [36, 21]
    table = torch.tensor([[1], [0]], dtype=torch.int32)
    k0 = torch.randn(total[0], HKV, D, generator=g).to(torch.bfloat16)
    v0 = torch.randn(total[0], HKV, D, generator=g).to(torch.bfloat16)
    k1 = torch.randn(total[1], HKV, D, generator=g).to(torch.bfloat16)
    v1 = torch.randn(total[1], HKV, D, generator=g).to(torch.bfloat16)
    q1 = torch.randn(16, HQ, D, generator=g).to(torch.bfloat16)     # step 1: 8 + 8 queries
    q2 = torch.randn(16, HQ, D, generator=g).to(torch.bfloat16)     # step 2
    kc = torch.zeros(2, P, HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[1, :36], vc[1, :36] = k0, v0
    kc[0, :21], vc[0, :21] = k1, v1
    cu_q = torch.tensor([0, 8, 16], dtype=torch.int32)
    out1 = OA.varlen_prefill(q1, kc, vc, cu_q, torch.tensor([0, 28, 41], dtype=torch.int32),
                             table, D ** -0.5)
    out2 = OA.varlen_prefill(q2, kc, vc, cu_q, torch.tensor([0, 36, 57], dtype=torch.int32),
                             table, D ** -0.5)
    save_file({"k0": k0, "v0": v0, "k1": k1, "v1": v1, "q_step1": q1, "q_step2": q2,
               "block_tables": table, "cu_q": cu_q,
               "cu_k_step1": torch.tensor([0, 28, 41], dtype=torch.int32),
               "cu_k_step2": torch.tensor([0, 36, 57], dtype=torch.int32),
               "out_step1_fp32": out1.contiguous(), "out_step2_fp32": out2.contiguous()},
              os.path.join(HERE, "prefill_small.safetensors"))


# ---------------------------------------------------------------------------
def grpo_small():
    """4 sequences (prompts 0,0,1,1) x 16 tokens, vocab 1024, logits N(0, 2)."""
    g = torch.Generator().manual_seed(303)
    logits = (2.0 * torch.randn(4, 16, 1024, generator=g)).to(torch.bfloat16)
    ids = torch.multinomial(torch.softmax(logits.float().view(-1, 1024), -1), 1,
                            generator=g).view(4, 16)
    lens = torch.tensor([16, 9, 1, 12])
    mask = (torch.arange(16)[None] < lens[:, None]).float()
    rewards = torch.tensor([1.0, 0.0, 1.0, 1.0])
    prompt_ids = torch.tensor([0, 0, 1, 1])
    lp, lse = OG.logprob_gather(logits, ids)
    old = (lp + 0.3 * torch.randn(4, 16, generator=g)) * mask     # some ratios clip at eps 0.2
    t = {"logits": logits, "ids": ids, "mask": mask, "old_lp": old.contiguous(),
         "rewards": rewards, "prompt_ids": prompt_ids, "lp": lp.contiguous(),
         "lse": lse.contiguous()}
    for eps_name, eps in (("1e-8", 1e-8), ("1e-4", 1e-4)):
        for red in ("token", "seq"):
            r = OG.fused_loss_step(logits, ids, old, mask, rewards, prompt_ids, eps, 0.2, red)
            t[f"adv_eps{eps_name}"] = r["adv"].contiguous()
            t[f"loss_{red}_eps{eps_name}"] = r["loss"].reshape(1)
            t[f"dlp_{red}_eps{eps_name}"] = r["dlp"].contiguous()
    save_file(t, os.path.join(HERE, "grpo_small.safetensors"))


# ---------------------------------------------------------------------------
def block_manager_trace():
    pkg = importlib.import_module("qwen3-naive-inference_amd")
    BM, Seq = pkg.paged.BlockManager, pkg.paged.Sequence
    g = torch.Generator().manual_seed(404)
    prefix = torch.randint(0, 151936, (512,), generator=g).tolist()
    tails = {n: torch.randint(0, 151936, (k,), generator=g).tolist()
             for n, k in (("A", 100), ("B", 300), ("C", 10))}
    prompts = {"A": prefix + tails["A"], "B": prefix + tails["B"], "C": prefix + tails["C"],
               "D": prefix + tails["B"]}
    bm = BM(8)
    seqs = {}
    steps = []

    def snap(op):
        steps.append({
            "op": op,
            "tables": {k: list(s.block_table) for k, s in seqs.items()},
            "kv_len": {k: s.kv_len for k, s in seqs.items()},
            "ref_count": list(bm.ref_count),
            "free": list(bm.free),
            "hashed_blocks": sorted(b for b in range(8) if bm.block_hash[b] != -1),
        })

    def prefill(name):
        s = seqs[name]
        s.num_scheduled_tokens = s.num_tokens - s.kv_len
        s.kv_len = s.num_tokens
        bm.hash_blocks(s)
        s.num_scheduled_tokens = 0

    for name in ("A", "B"):
        seqs[name] = Seq(prompts[name])
        bm.allocate(seqs[name])
        snap(["allocate", name])
        prefill(name)
        snap(["prefill", name])
    s = seqs["A"]
    for i in range(156):                          # decode A from 612 to 768 keys
        s.append_token(i)
        s.kv_len += 1
    bm.may_append(s)                              # 768 % 256 == 0: a new page
    snap(["decode_to", "A", 768])
    bm.deallocate(seqs.pop("A").block_table)
    snap(["deallocate", "A"])
    seqs["C"] = Seq(prompts["C"])
    bm.allocate(seqs["C"])
    snap(["allocate", "C"])
    bm.deallocate(seqs.pop("B").block_table)
    snap(["deallocate", "B"])
    seqs["D"] = Seq(prompts["D"])
    bm.allocate(seqs["D"])
    snap(["allocate", "D"])

    # Hand-derived expectations (free list [0..7] popped from the end).
    by_op = {tuple(x["op"][:2]): x for x in steps}
    assert by_op[("allocate", "A")]["tables"]["A"] == [7, 6, 5]
    assert by_op[("allocate", "B")]["tables"]["B"] == [7, 6, 4, 3]        # 2 prefix hits
    assert by_op[("allocate", "B")]["kv_len"]["B"] == 512
    assert by_op[("prefill", "B")]["hashed_blocks"] == [4, 6, 7]
    assert by_op[("decode_to", "A")]["tables"]["A"] == [7, 6, 5, 2]
    assert by_op[("deallocate", "A")]["free"] == [0, 1, 5, 2]
    assert by_op[("allocate", "C")]["tables"]["C"] == [7, 6, 2]
    assert by_op[("deallocate", "B")]["free"] == [0, 1, 5, 4, 3]
    assert by_op[("allocate", "D")]["tables"]["D"] == [7, 6, 4, 3]        # 4 revived, 3 popped
    assert by_op[("allocate", "D")]["kv_len"]["D"] == 768
    assert by_op[("allocate", "D")]["ref_count"] == [0, 0, 1, 1, 1, 0, 2, 2]   # C holds 2
    assert by_op[("allocate", "D")]["free"] == [0, 1, 5]
    with open(os.path.join(HERE, "block_manager_trace.json"), "w") as f:
        json.dump({"num_blocks": 8, "block_size": 256, "prompts": prompts, "steps": steps}, f)


if __name__ == "__main__":
    torch.set_num_threads(1)
    config1()
    decode_small()
    prefill_small()
    grpo_small()
    block_manager_trace()
    print("fixtures written to", HERE)
