"""Pins the oracle's paged-KV bookkeeping and KV store (CPU)."""
import random

import pytest
import torch

from oracle import paged


def test_hash_known_answers():
    # Hand-computed from h = ((h << 5) + h) ^ t, h0 = 0 (qwen3_naive.py:264-267):
    # [1, 2]: h = 0*33 ^ 1 = 1; h = 1*33 ^ 2 = 35.
    assert paged.compute_hash([1, 2]) == 35
    # [7]: 0*33 ^ 7 = 7.  Chained from prefix 35: 35*33 ^ 7 = 1155 ^ 7 = 1156.
    assert paged.compute_hash([7]) == 7
    assert paged.compute_hash([7], 35) == 1156
    assert paged.compute_hash([]) == 0
    # prefix -1 means "no prefix" and equals prefix 0.
    assert paged.compute_hash([5, 6], -1) == paged.compute_hash([5, 6], 0)


def test_hash_wraps_like_uint64():
    rng = random.Random(0)
    for _ in range(50):
        toks = [rng.randrange(151936) for _ in range(rng.randrange(1, 300))]
        prefix = rng.choice([-1, rng.randrange(1 << 64)])
        assert paged.compute_hash(toks, prefix) == paged.compute_hash_u64(toks, prefix)
    # 13 steps of *33 overflow 64 bits for a large seed: both must agree.
    big = (1 << 63) + 12345
    assert paged.compute_hash([1] * 13, big) == paged.compute_hash_u64([1] * 13, big)
    assert paged.compute_hash([1] * 13, big) < (1 << 64)


def test_chained_hash_distinguishes_prefixes():
    a = paged.compute_hash([1, 2, 3])
    b = paged.compute_hash([1, 2, 4])
    assert paged.compute_hash([9], a) != paged.compute_hash([9], b)


def test_decode_slot_closed_form():
    bt = [5, 2, 9]
    assert paged.decode_slot(bt, 0) == 5 * 256
    assert paged.decode_slot(bt, 255) == 5 * 256 + 255
    assert paged.decode_slot(bt, 256) == 2 * 256
    assert paged.decode_slot(bt, 700) == 9 * 256 + 700 - 512


def test_token_slots_block_by_block():
    # The reference walks blocks [start//B, ceil(end/B)) and emits runs; the
    # per-position closed form must produce the same runs.
    bt = [3, 7, 1, 4]
    for start, end in [(0, 1), (0, 256), (100, 700), (256, 512), (511, 513), (300, 1024)]:
        runs = []
        sb, eb = start // 256, (end + 255) // 256
        for blk in range(sb, eb):
            s0 = bt[blk] * 256 + (start % 256 if blk == sb else 0)
            s1 = bt[blk] * 256 + (end - blk * 256 if blk == eb - 1 else 256)
            runs += list(range(s0, s1))
        assert paged.token_slots(bt, start, end) == runs


def test_prepare_step_integer_invariants():
    # Mirrors the integer assertions of the reference's chunked-prefill tests
    # (test_chunked_prefill.py:201-204 and :293-303).
    seqs = [
        dict(token_ids=list(range(40)), kv_len=39, num_scheduled_tokens=1, block_table=[0]),
        dict(token_ids=list(range(12)), kv_len=11, num_scheduled_tokens=1, block_table=[1]),
        dict(token_ids=list(range(1200)), kv_len=0, num_scheduled_tokens=512,
             block_table=[2, 3, 4, 5, 6]),
    ]
    st = paged.prepare_step(seqs)
    assert st["cu_seqlens_q"] == [0, 1, 2, 514]
    assert st["cu_seqlens_k"] == [0, 40, 52, 564]
    assert st["max_seqlen_q"] == 512 and st["max_seqlen_k"] == 512
    assert len(st["block_tables"]) == 3 and all(len(r) == 5 for r in st["block_tables"])
    assert st["block_tables"][0] == [0, -1, -1, -1, -1]
    assert st["block_mapping"][:2] == [39, 256 + 11]
    assert st["block_mapping"][2:] == [2 * 256 + p if p < 256 else 3 * 256 + p - 256
                                       for p in range(512)]
    assert st["positions"][:2] == [39, 11]


def test_store_brute_force():
    g = torch.Generator().manual_seed(3)
    key = torch.randn(6, 2, 4, generator=g).to(torch.bfloat16)
    val = torch.randn(6, 2, 4, generator=g).to(torch.bfloat16)
    kc = torch.zeros(3, 4, 2, 4, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = [5, -1, 0, 11, 7, -1]
    paged.store_kvcache(key, val, kc, vc, slots)
    kf, vf = kc.view(-1, 8), vc.view(-1, 8)
    written = set()
    for i, s in enumerate(slots):
        if s >= 0:
            assert torch.equal(kf[s], key[i].reshape(8))
            assert torch.equal(vf[s], val[i].reshape(8))
            written.add(s)
    for s in range(12):
        if s not in written:
            assert kf[s].abs().sum() == 0 and vf[s].abs().sum() == 0


@pytest.mark.parametrize("bad", [[0, 1, 2], [1, 0, 3]])
def test_block_tables_padding(bad):
    out = paged.block_tables([bad, [4]])
    assert out[1] == [4, -1, -1]
