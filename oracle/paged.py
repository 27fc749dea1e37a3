"""Paged-KV bookkeeping and the KV store, restated on the CPU.

Reference: qwen3_naive.py
  _store_kvcache_kernel / store_kvcache  :20-41
  BlockManager.compute_hash              :261-267
  _prepare_step block_mapping / cu_seqlens :1147-1199
  _build_block_tables                    :1201-1205
  _prepare_decode slot_mapping           :1207-1225
"""
from __future__ import annotations

import numpy as np
import torch

BLOCK_SIZE = 256
MASK64 = (1 << 64) - 1


def compute_hash(token_ids, prefix_hash: int = -1) -> int:
    """Chained djb2-style hash over a block's token ids (qwen3_naive.py:261-267).

    ``h = ((h << 5) + h) ^ t`` per token starting from the previous block's
    hash (0 for the first block); the result is reduced to 64 bits.  Python
    ints are unbounded, so reducing only at the end equals uint64 wrap-around
    at every step.
    """
    h = prefix_hash if prefix_hash != -1 else 0
    for t in token_ids:
        h = ((h << 5) + h) ^ int(t)
    return h & MASK64


def compute_hash_u64(token_ids, prefix_hash: int = -1) -> int:
    """Same hash with explicit uint64 arithmetic at every step (numpy)."""
    h = np.uint64(prefix_hash if prefix_hash != -1 else 0)
    with np.errstate(over="ignore"):
        for t in token_ids:
            h = np.uint64((h << np.uint64(5)) + h) ^ np.uint64(int(t) & MASK64)
    return int(h)


def decode_slot(block_table: list[int], kv_len: int, block_size: int = BLOCK_SIZE) -> int:
    """Slot of the token written at position ``kv_len`` (qwen3_naive.py:1216-1223)."""
    return block_table[kv_len // block_size] * block_size + kv_len % block_size


def token_slots(block_table: list[int], start: int, end: int,
                block_size: int = BLOCK_SIZE) -> list[int]:
    """Per-token slots for positions [start, end) (qwen3_naive.py:1176-1187).

    The reference builds the list block by block; per position it equals
    ``block_table[p // B] * B + p % B``.
    """
    return [block_table[p // block_size] * block_size + p % block_size for p in range(start, end)]


def prepare_step(seqs) -> dict:
    """Varlen step inputs for sequences given as dicts with keys
    ``token_ids, kv_len, num_scheduled_tokens, block_table``
    (qwen3_naive.py:1147-1199)."""
    input_ids, positions, cu_q, cu_k, mapping = [], [], [0], [0], []
    max_q = max_k = 0
    for s in seqs:
        start = s["kv_len"]
        end = start + s["num_scheduled_tokens"]
        input_ids += list(s["token_ids"][start:end])
        positions += list(range(start, end))
        cu_q.append(cu_q[-1] + (end - start))
        cu_k.append(cu_k[-1] + end)
        max_q = max(max_q, end - start)
        max_k = max(max_k, end)
        mapping += token_slots(s["block_table"], start, end)
    return {"input_ids": input_ids, "positions": positions, "cu_seqlens_q": cu_q,
            "cu_seqlens_k": cu_k, "max_seqlen_q": max_q, "max_seqlen_k": max_k,
            "block_mapping": mapping, "block_tables": block_tables([s["block_table"] for s in seqs])}


def block_tables(tables: list[list[int]]) -> list[list[int]]:
    """-1-padded rectangular block tables (qwen3_naive.py:1201-1205)."""
    width = max(len(t) for t in tables)
    return [list(t) + [-1] * (width - len(t)) for t in tables]


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping) -> None:
    """In-place KV store (qwen3_naive.py:20-41): row ``slot`` of the flattened
    caches receives token i's ``[H*D]`` row; slot -1 is skipped.  Loops over
    tokens exactly as the reference launches one program per token."""
    n = key.shape[0]
    row = key.shape[1] * key.shape[2]
    kf = k_cache.view(-1, row)
    vf = v_cache.view(-1, row)
    slots = [int(s) for s in (slot_mapping.tolist() if torch.is_tensor(slot_mapping)
                              else slot_mapping)]
    for i in range(n):
        s = slots[i]
        if s == -1:
            continue
        kf[s] = key[i].reshape(row)
        vf[s] = value[i].reshape(row)
