"""Paged-KV bookkeeping for continuous batching: sequences, the block manager
with chained-hash prefix caching, and the per-step index tensors.

Behaviour follows qwen3-naive-inference's qwen3_naive.py:
  Sequence                 :191-237  per-request state, 256-token pages
  BlockManager             :240-375  free list + refcounts + prefix cache
  _prepare_step            :1147-1199 varlen inputs and per-token slots
  _build_block_tables      :1201-1205 -1-padded [B, W] tables
  _prepare_decode          :1207-1225 decode inputs and slots
The free-list order (pop from the end, freed blocks appended, reused cached
blocks removed in place) is kept, so block ids -- and therefore slots -- are
assigned exactly as the reference assigns them for the same operation
sequence.  Index tensors are built with numpy in one pass per step and sent
with one pinned, non-blocking copy each.
"""
from __future__ import annotations

import numpy as np
import torch

BLOCK_SIZE = 256
_MASK64 = (1 << 64) - 1


class Sequence:
    """One request: token ids, page table and KV progress (qwen3_naive.py:191-237)."""

    BLOCK_SIZE = BLOCK_SIZE

    def __init__(self, token_ids: list[int], sampling_params: dict | None = None):
        self.token_ids = list(token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        self.last_token = self.token_ids[-1]
        self.status = "WAITING"
        self.block_table: list[int] = []
        self.kv_len = 0                 # tokens whose K/V are in the cache
        self.num_scheduled_tokens = 0   # tokens computed this step
        sp = sampling_params or {}
        self.temperature = sp.get("temperature", 0.6)
        self.max_tokens = sp.get("max_tokens", 256)
        self.response_log_probs: list[float] = []

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)
        self.last_token = token_id

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def num_blocks(self) -> int:
        return (len(self.token_ids) + self.BLOCK_SIZE - 1) // self.BLOCK_SIZE

    def block(self, i: int) -> list[int]:
        s = i * self.BLOCK_SIZE
        return self.token_ids[s:min(s + self.BLOCK_SIZE, len(self.token_ids))]

    @property
    def num_completion_tokens(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens

    @property
    def unfinished(self) -> bool:
        return self.status != "FINISHED"

    @property
    def prompt_len(self) -> int:
        return self.num_prompt_tokens


class BlockManager:
    """Refcounted page allocator with a chained-hash prefix cache
    (qwen3_naive.py:240-375).

    A full page is shared when the hash of its tokens chained onto the hash of
    every earlier page matches a registered page *and* its token list is equal
    (collision guard).  Freed pages keep their hash so a later request with
    the same prefix can revive them; a page is only stripped of its hash when
    it is reallocated for other content.
    """

    def __init__(self, num_blocks: int, block_size: int = BLOCK_SIZE):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.free: list[int] = list(range(num_blocks))
        self.ref_count = [0] * num_blocks
        self.block_hash = [-1] * num_blocks
        self.block_tokens: list[list[int] | None] = [None] * num_blocks
        self.hash_to_block: dict[int, int] = {}

    @staticmethod
    def compute_hash(token_ids, prefix_hash: int = -1) -> int:
        h = 0 if prefix_hash == -1 else prefix_hash
        for t in token_ids:
            h = (h * 33) ^ t        # ((h << 5) + h) ^ t
        return h & _MASK64

    def _take_free(self, blk: int | None = None) -> int:
        """Pop the last free page (or remove ``blk``) and strip any old hash."""
        if blk is None:
            blk = self.free.pop()
        old = self.block_hash[blk]
        if old != -1:
            if self.hash_to_block.get(old) == blk:
                del self.hash_to_block[old]
            self.block_hash[blk] = -1
            self.block_tokens[blk] = None
        self.ref_count[blk] = 1
        return blk

    def allocate(self, seq: Sequence) -> None:
        assert not seq.block_table, "sequence already holds pages"
        h = -1
        cached = 0
        for i in range(seq.num_blocks - 1):  # the last (possibly partial) page is never shared
            toks = seq.block(i)
            h = self.compute_hash(toks, h)
            blk = self.hash_to_block.get(h, -1)
            if blk == -1 or self.block_tokens[blk] != toks:
                break
            cached += 1
            if self.ref_count[blk] == 0:      # freed but still hashed: revive it
                self.free.remove(blk)
            self.ref_count[blk] += 1
            seq.block_table.append(blk)
        for _ in range(cached, seq.num_blocks):
            seq.block_table.append(self._take_free())
        seq.kv_len = cached * self.block_size

    def deallocate(self, block_table: list[int]) -> None:
        for b in block_table:
            self.ref_count[b] -= 1
            if self.ref_count[b] == 0:
                self.free.append(b)           # hash kept for reuse

    def can_append(self, seq: Sequence) -> bool:
        return seq.kv_len % self.block_size != 0 or len(self.free) > 0

    def may_append(self, seq: Sequence) -> None:
        if seq.kv_len % self.block_size == 0:
            seq.block_table.append(self._take_free())

    def hash_blocks(self, seq: Sequence) -> None:
        """Register the pages completed by this step (prefill chunks)."""
        start = (seq.kv_len - seq.num_scheduled_tokens) // self.block_size
        end = seq.kv_len // self.block_size
        if start >= end:
            return
        h = self.block_hash[seq.block_table[start - 1]] if start > 0 else -1
        for i in range(start, end):
            blk = seq.block_table[i]
            toks = seq.block(i)
            h = self.compute_hash(toks, h)
            self.block_hash[blk] = h
            self.block_tokens[blk] = toks
            self.hash_to_block[h] = blk

    @property
    def available(self) -> int:
        return len(self.free)


# ---------------------------------------------------------------------------
def _to_device(arr: np.ndarray, device) -> torch.Tensor:
    t = torch.from_numpy(arr)
    if device is None or torch.device(device).type == "cpu":
        return t
    return t.pin_memory().to(device, non_blocking=True)


def build_block_tables(seqs: list[Sequence], width: int | None = None) -> np.ndarray:
    """-1-padded int32 [B, W] page tables (W = longest table unless given)."""
    w = max(len(s.block_table) for s in seqs) if width is None else width
    out = np.full((len(seqs), w), -1, dtype=np.int32)
    for i, s in enumerate(seqs):
        n = min(len(s.block_table), w)
        out[i, :n] = s.block_table[:n]
    return out


def token_slots(table: list[int], start: int, end: int, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Slots of positions [start, end): table[p // B] * B + p % B."""
    p = np.arange(start, end, dtype=np.int64)
    return (np.asarray(table, dtype=np.int64)[p // block_size] * block_size + p % block_size).astype(np.int32)


def prepare_step(seqs: list[Sequence], device=None, block_size: int = BLOCK_SIZE):
    """Varlen step inputs (qwen3_naive.py:1147-1199).

    Returns (input_ids int64, positions int64, cu_seqlens_q int32, cu_seqlens_k
    int32, max_seqlen_q, max_seqlen_k, block_mapping int32, block_tables int32).
    """
    n_new = [s.num_scheduled_tokens for s in seqs]
    starts = [s.kv_len for s in seqs]
    ids, pos, slots = [], [], []
    cu_q = np.zeros(len(seqs) + 1, dtype=np.int32)
    cu_k = np.zeros(len(seqs) + 1, dtype=np.int32)
    for i, s in enumerate(seqs):
        st, en = starts[i], starts[i] + n_new[i]
        ids.append(np.asarray(s.token_ids[st:en], dtype=np.int64))
        pos.append(np.arange(st, en, dtype=np.int64))
        slots.append(token_slots(s.block_table, st, en, block_size))
        cu_q[i + 1] = cu_q[i] + (en - st)
        cu_k[i + 1] = cu_k[i] + en
    max_q = max(n_new) if seqs else 0
    max_k = max(st + n for st, n in zip(starts, n_new)) if seqs else 0
    cat = lambda xs, dt: np.concatenate(xs) if xs else np.zeros(0, dtype=dt)
    return (_to_device(cat(ids, np.int64), device), _to_device(cat(pos, np.int64), device),
            _to_device(cu_q, device), _to_device(cu_k, device), max_q, max_k,
            _to_device(cat(slots, np.int32), device),
            _to_device(build_block_tables(seqs), device))


def fill_decode_inputs(seqs: list[Sequence], ids: np.ndarray, pos: np.ndarray, ctx: np.ndarray,
                       slot: np.ndarray, tables: np.ndarray, block_size: int = BLOCK_SIZE) -> None:
    """The decode inputs of ``prepare_decode`` written into rows ``0 .. len(seqs)-1``
    of caller-provided host arrays (``tables`` is ``[rows, W]``, -1 past each
    table); rows past ``len(seqs)`` are left to the caller."""
    n = len(seqs)
    ids[:n] = np.fromiter((s.last_token for s in seqs), dtype=np.int64, count=n)
    pos[:n] = np.fromiter((s.num_tokens - 1 for s in seqs), dtype=np.int64, count=n)
    ctx[:n] = np.fromiter((s.kv_len for s in seqs), dtype=np.int32, count=n)
    slot[:n] = np.fromiter((s.block_table[s.kv_len // block_size] * block_size + s.kv_len % block_size
                            for s in seqs), dtype=np.int32, count=n)
    tables[:n] = -1
    w = tables.shape[1]
    for i, sq in enumerate(seqs):
        m = min(len(sq.block_table), w)
        tables[i, :m] = sq.block_table[:m]


def near_equal_contexts(ctx: np.ndarray) -> bool:
    """True when every row's key count (context + 1) is within 10% of the
    rows' mean: the decode attention then runs one whole (sequence, head
    group) unit per workgroup with no merge, since the longest unit is not
    much longer than a balanced share.  ``ctx`` holds the context lengths of
    every row the kernel sees (padding rows included)."""
    if len(ctx) == 0:
        return False
    keys = ctx.astype(np.int64) + 1
    return 10 * int(keys.max()) * len(keys) <= 11 * int(keys.sum())


def prepare_decode(seqs: list[Sequence], device=None, block_size: int = BLOCK_SIZE,
                   width: int | None = None):
    """Decode inputs (qwen3_naive.py:1207-1225): last token, its position
    (num_tokens - 1), context_lens = kv_len, -1-padded block tables and the
    slot of position kv_len."""
    ids = np.fromiter((s.last_token for s in seqs), dtype=np.int64, count=len(seqs))
    pos = np.fromiter((s.num_tokens - 1 for s in seqs), dtype=np.int64, count=len(seqs))
    ctx = np.fromiter((s.kv_len for s in seqs), dtype=np.int32, count=len(seqs))
    slot = np.fromiter((s.block_table[s.kv_len // block_size] * block_size + s.kv_len % block_size
                        for s in seqs), dtype=np.int32, count=len(seqs))
    return (_to_device(ids, device), _to_device(pos, device), _to_device(ctx, device),
            _to_device(build_block_tables(seqs, width), device), _to_device(slot, device))
