"""Seeded synthetic inputs for the five benchmark configurations.

Shapes follow the Qwen3-0.6B attention (16 query heads, 8 KV heads, head_dim
128, 256-token pages) and the GRPO loss step (32 x 512 rows, vocab 151936).
Integer structure (lengths, permutations, block tables) is drawn on the CPU
from ``torch.Generator().manual_seed(seed)`` so it is identical on every
machine; large float tensors are drawn on ``device`` from a generator seeded
the same way.
"""
from __future__ import annotations

import math

import torch

HQ, HKV, D, P = 16, 8, 128, 256
VOCAB = 151936


def _gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn_bf16(shape, g, device, scale=1.0):
    return (torch.randn(shape, generator=g, device=device) * scale).to(torch.bfloat16)


# ---------------------------------------------------------------------------
def decode_one_layer(seed: int = 0, device="cpu", ctx=(37, 256, 300, 700), num_blocks=16):
    """Config 1: one paged decode step of one attention layer.

    q [4,16,128], new K/V [4,8,128], pools [16,256,8,128], all N(0,1) bf16;
    block_tables = randperm(16).view(4,4); the new token of sequence b is
    stored at slot bt[b, ctx//256]*256 + ctx%256 and attention covers ctx+1 keys.
    """
    g = _gen(seed, "cpu")
    bsz = len(ctx)
    q = _randn_bf16((bsz, HQ, D), g, "cpu")
    k_new = _randn_bf16((bsz, HKV, D), g, "cpu")
    v_new = _randn_bf16((bsz, HKV, D), g, "cpu")
    k_cache = _randn_bf16((num_blocks, P, HKV, D), g, "cpu")
    v_cache = _randn_bf16((num_blocks, P, HKV, D), g, "cpu")
    perm = torch.randperm(num_blocks, generator=g)
    width = num_blocks // bsz
    bt = perm.view(bsz, width).to(torch.int32)
    ctx_t = torch.tensor(ctx, dtype=torch.int32)
    slots = torch.tensor([int(bt[b, c // P]) * P + c % P for b, c in enumerate(ctx)],
                         dtype=torch.int32)
    out = dict(q=q, k_new=k_new, v_new=v_new, k_cache=k_cache, v_cache=v_cache,
               block_tables=bt, context_lens=ctx_t, slot_mapping=slots,
               cache_seqlens=ctx_t + 1, scale=D ** -0.5)
    return {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in out.items()}


def decode_batch(seed: int = 0, device="cpu", batch=64, ctx_lo=1024, ctx_hi=4096,
                 layers: int = 1, extra_blocks: int = 0):
    """Config 3 attention inputs: B=64 sequences, ctx ~ U{1024..4096}.

    Each sequence needs ceil((ctx+1)/256) pages; the pool holds exactly the
    pages needed (+extra) and the block tables are a shuffled permutation of
    it.  ``layers`` independent K/V pools ([layers, NB, 256, 8, 128]) let a
    benchmark rotate layers so the 256 MB Infinity Cache cannot hold the data.
    """
    g = _gen(seed, "cpu")
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=g, dtype=torch.int64)
    need = [(int(c) + 1 + P - 1) // P for c in ctx]
    nb = sum(need) + extra_blocks
    perm = torch.randperm(nb, generator=g)
    width = max(need)
    bt = torch.full((batch, width), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    gd = _gen(seed + 1, device)
    q = _randn_bf16((batch, HQ, D), gd, device)
    shape = (layers, nb, P, HKV, D) if layers > 1 else (nb, P, HKV, D)
    k_cache = _randn_bf16(shape, gd, device)
    v_cache = _randn_bf16(shape, gd, device)
    return dict(q=q, k_cache=k_cache, v_cache=v_cache, block_tables=bt.to(device),
                context_lens=ctx.to(torch.int32).to(device),
                cache_seqlens=(ctx + 1).to(torch.int32).to(device), scale=D ** -0.5,
                num_blocks=nb, kv_bytes=int(sum(int(c) + 1 for c in ctx)) * HKV * D * 2 * 2)


def decode_kv_bytes(cache_seqlens) -> int:
    """Algorithmic K+V bytes read by one decode-attention launch."""
    lens = cache_seqlens.tolist() if torch.is_tensor(cache_seqlens) else cache_seqlens
    return int(sum(int(x) for x in lens)) * HKV * D * 2 * 2


# ---------------------------------------------------------------------------
def grpo_loss_step(seed: int = 0, device="cpu", n_prompts=4, group=8, n_tok=512, vocab=VOCAB,
                   len_lo=64, len_hi=512, logit_std=2.0, old_noise=0.05, chunk_rows=1024):
    """Config 2: GRPO loss step inputs.

    logits = N(0, logit_std^2) bf16 [R, T, V]; ids ~ Categorical(softmax(logits))
    drawn with the Gumbel-max construction per row; rewards ~ Bernoulli(0.5);
    prompt_ids = [0]*group + [1]*group + ...; mask[b, t] = t < len_b with
    len_b ~ U{len_lo..len_hi}; old = new + old_noise * N(0,1) where ``new`` is
    the exact fp32 log-probability of the sampled id (torch.log_softmax).
    """
    r = n_prompts * group
    gc = _gen(seed, "cpu")
    rewards = torch.bernoulli(torch.full((r,), 0.5), generator=gc)
    lens = torch.randint(len_lo, len_hi + 1, (r,), generator=gc)
    mask = (torch.arange(n_tok)[None, :] < lens[:, None]).float()
    prompt_ids = torch.arange(n_prompts).repeat_interleave(group)
    gd = _gen(seed + 1, device)
    logits = torch.empty((r, n_tok, vocab), dtype=torch.bfloat16, device=device)
    ids = torch.empty((r, n_tok), dtype=torch.int64, device=device)
    new = torch.empty((r, n_tok), dtype=torch.float32, device=device)
    flat = logits.view(-1, vocab)
    fids = ids.view(-1)
    fnew = new.view(-1)
    for s in range(0, r * n_tok, chunk_rows):
        e = min(s + chunk_rows, r * n_tok)
        x = torch.randn((e - s, vocab), generator=gd, device=device) * logit_std
        xb = x.to(torch.bfloat16)
        flat[s:e] = xb
        xf = xb.float()
        u = torch.rand((e - s, vocab), generator=gd, device=device).clamp_(1e-20, 1.0)
        pick = torch.argmax(xf - torch.log(-torch.log(u)), dim=-1)
        fids[s:e] = pick
        fnew[s:e] = torch.log_softmax(xf, dim=-1).gather(-1, pick[:, None])[:, 0]
        del x, xf, u
    old = new + old_noise * torch.randn((r, n_tok), generator=gd, device=device)
    return dict(logits=logits, ids=ids, old_lp=old, new_lp=new, mask=mask.to(device),
                rewards=rewards.to(device), prompt_ids=prompt_ids.to(device),
                lens=lens, logit_bytes=r * n_tok * vocab * 2)


# ---------------------------------------------------------------------------
def prefix_prefill_chunks(seed: int = 0, n_seq=16, prefix=512, suf_lo=256, suf_hi=2048,
                          chunk=512):
    """Config 4 schedule: shared cached prefix + per-sequence suffix in chunks.

    Returns the per-sequence suffix lengths and, per step, the list of
    (seq, kv_before, n_new) triples: every unfinished sequence contributes its
    next chunk of at most ``chunk`` tokens.
    """
    g = _gen(seed, "cpu")
    suf = torch.randint(suf_lo, suf_hi + 1, (n_seq,), generator=g).tolist()
    done = [0] * n_seq
    steps = []
    while any(done[b] < suf[b] for b in range(n_seq)):
        step = []
        for b in range(n_seq):
            if done[b] < suf[b]:
                n = min(chunk, suf[b] - done[b])
                step.append((b, prefix + done[b], n))
                done[b] += n
        steps.append(step)
    pairs = sum(sum(p + 1 for p in range(prefix, prefix + s)) for s in suf)
    return dict(suffix=suf, steps=steps, causal_pairs=pairs, prefix=prefix,
                flops_per_layer=4 * HQ * D * pairs)


def prefill_step_inputs(seed: int, step, prefix_blocks, n_blocks_total, device="cpu"):
    """Attention inputs for one chunk step of ``prefix_prefill_chunks``.

    Every sequence's block table starts with the shared ``prefix_blocks`` and
    continues with its own pages (sequence b owns a contiguous run of a
    shuffled page permutation).  Returns q, cu_seqlens_q/k, block_tables.
    """
    g = _gen(seed + 7, "cpu")
    perm = torch.randperm(n_blocks_total, generator=g).tolist()
    perm = [p for p in perm if p not in set(prefix_blocks)]
    max_blocks = 0
    tables = []
    cu_q, cu_k = [0], [0]
    for (b, kv_before, n) in step:
        total = kv_before + n
        nblk = (total + P - 1) // P
        own = nblk - len(prefix_blocks)
        start = b * 16
        tables.append(list(prefix_blocks) + perm[start:start + own])
        max_blocks = max(max_blocks, nblk)
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + total)
    bt = torch.full((len(step), max_blocks), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    gd = _gen(seed + 11, device)
    q = _randn_bf16((cu_q[-1], HQ, D), gd, device)
    return dict(q=q, cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=device),
                cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=device),
                block_tables=bt.to(device), max_seqlen_q=max(n for _, _, n in step),
                max_seqlen_k=max(kv + n for _, kv, n in step))


def causal_pairs(cu_q, cu_k) -> int:
    """Number of unmasked (query, key) pairs of a bottom-right causal varlen step."""
    total = 0
    for b in range(len(cu_q) - 1):
        lq = int(cu_q[b + 1]) - int(cu_q[b])
        lk = int(cu_k[b + 1]) - int(cu_k[b])
        off = lk - lq
        total += sum(min(lk, i + off + 1) for i in range(lq))
    return total


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["decode_one_layer", "decode_batch", "decode_kv_bytes", "grpo_loss_step",
           "prefix_prefill_chunks", "prefill_step_inputs", "causal_pairs", "ceil_div", "math"]
