"""Paged attention restated on the CPU.

Reference call sites (qwen3_naive.py):
  decode : flash_attn_with_kvcache(q[:,None], k_cache, v_cache,
           cache_seqlens=context_lens+1, block_table, softmax_scale, causal=True)  :672-680
  prefill: flash_attn_varlen_func(q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k,
           max_seqlen_q, max_seqlen_k, softmax_scale, causal=True, block_table)    :631-637
flash-attn itself is a third-party dependency that is not in the reference
tree and has no pinned version; its semantics are restated from its public
documentation: keys of sequence b are rows 0..L_b-1 gathered through the
block table (row j at page block_table[b, j // 256], offset j % 256); causal
masking is aligned to the bottom-right corner, so query i of Lq new tokens
sees keys j <= i + Lk - Lq; query head h reads KV head h // (Hq / Hkv).

Two arithmetic modes:
  "fp32"       exact-math truth: fp32 scores, softmax and PV (float64 optional).
  "bf16_eager" the reference's own eager attention (qwen3_naive.py:496-507,
               573-589): bf16 q@k^T, bf16 scale, fp32 softmax cast to bf16,
               bf16 PV, GQA through repeat_interleave (:513-518).
"""
from __future__ import annotations

import torch

BLOCK_SIZE = 256


def gather_pages(cache: torch.Tensor, table_row, length: int) -> torch.Tensor:
    """Rows 0..length-1 of one sequence from a [NB, P, Hkv, D] paged cache."""
    p = cache.shape[1]
    table = [int(x) for x in (table_row.tolist() if torch.is_tensor(table_row) else table_row)]
    pos = torch.arange(length)
    blocks = torch.tensor([table[j // p] for j in range(length)], dtype=torch.long)
    return cache[blocks, pos % p]


def _attend(q, k, v, scale, causal_offset, mode, dtype=torch.float32):
    """q [Lq, Hq, D], k/v [Lk, Hkv, D] -> [Lq, Hq, D].

    ``causal_offset`` = Lk - Lq for bottom-right causal masking, None for no mask.
    """
    lq, hq, d = q.shape
    lk, hkv, _ = k.shape
    rep = hq // hkv
    if mode == "fp32":
        qf = q.to(dtype).permute(1, 0, 2)                       # [Hq, Lq, D]
        kf = k.to(dtype).repeat_interleave(rep, dim=1).permute(1, 0, 2)
        vf = v.to(dtype).repeat_interleave(rep, dim=1).permute(1, 0, 2)
        s = (qf @ kf.transpose(1, 2)) * scale
        if causal_offset is not None:
            i = torch.arange(lq)[:, None]
            j = torch.arange(lk)[None, :]
            s = s.masked_fill(j > i + causal_offset, float("-inf"))
        p = torch.softmax(s, dim=-1)
        return (p @ vf).permute(1, 0, 2)
    if mode == "bf16_eager":
        qb = q.to(torch.bfloat16).permute(1, 0, 2)
        kb = k.to(torch.bfloat16).repeat_interleave(rep, dim=1).permute(1, 0, 2)
        vb = v.to(torch.bfloat16).repeat_interleave(rep, dim=1).permute(1, 0, 2)
        s = (qb @ kb.transpose(1, 2).contiguous()) * scale
        if causal_offset is not None:
            i = torch.arange(lq)[:, None]
            j = torch.arange(lk)[None, :]
            s = s.masked_fill(j > i + causal_offset, float("-inf"))
        w = torch.softmax(s.float(), dim=-1).to(torch.bfloat16)
        return (w @ vb).permute(1, 0, 2)
    raise ValueError(mode)


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 cache_seqlens, block_table, scale: float, mode: str = "fp32",
                 dtype=torch.float32) -> torch.Tensor:
    """One query per sequence: q [B, Hq, D] -> out [B, Hq, D] (fp32 result)."""
    bsz = q.shape[0]
    lens = [int(x) for x in (cache_seqlens.tolist() if torch.is_tensor(cache_seqlens)
                             else cache_seqlens)]
    out = torch.zeros(q.shape, dtype=dtype if mode == "fp32" else torch.float32)
    for b in range(bsz):
        if lens[b] <= 0:
            continue
        k = gather_pages(k_cache, block_table[b], lens[b])
        v = gather_pages(v_cache, block_table[b], lens[b])
        out[b] = _attend(q[b:b + 1], k, v, scale, None, mode, dtype)[0].to(out.dtype)
    return out


def varlen_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   cu_seqlens_q, cu_seqlens_k, block_table, scale: float,
                   mode: str = "fp32", dtype=torch.float32) -> torch.Tensor:
    """Varlen paged causal attention: q [Tq, Hq, D] -> out [Tq, Hq, D] (fp32)."""
    cq = [int(x) for x in (cu_seqlens_q.tolist() if torch.is_tensor(cu_seqlens_q) else cu_seqlens_q)]
    ck = [int(x) for x in (cu_seqlens_k.tolist() if torch.is_tensor(cu_seqlens_k) else cu_seqlens_k)]
    out = torch.zeros(q.shape, dtype=dtype if mode == "fp32" else torch.float32)
    for b in range(len(cq) - 1):
        lq = cq[b + 1] - cq[b]
        lk = ck[b + 1] - ck[b]
        if lq == 0:
            continue
        k = gather_pages(k_cache, block_table[b], lk)
        v = gather_pages(v_cache, block_table[b], lk)
        o = _attend(q[cq[b]:cq[b + 1]], k, v, scale, lk - lq, mode, dtype)
        out[cq[b]:cq[b + 1]] = o.to(out.dtype)
    return out
