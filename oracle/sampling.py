"""Sampling step of the rollout (test infrastructure only).

Follows qwen3_naive.py:1413-1423 (generate_continuous) and :1636-1650
(generate_continuous_with_logprobs) for top_k = None:
    x = logits.float() / T;  tok ~ Categorical(softmax(x));  lp = log_softmax(x)[tok]

The draw is restated as Gumbel-max with the uniforms of Philox4x32-10
(Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
SC 2011): element i of row r uses word i % 4 of the block at counter
(i / 4, r, offset_lo, offset_hi) and key (seed_lo, seed_hi), mapped to
U = ((w >> 8) + 0.5) / 2^24.  ``gumbel_scores`` gives x_i log2(e) - log2(E_i log2(e)),
E_i = -ln U_i, in float64, so a kernel that follows the same stream picks the
same argmax wherever the top two scores are not within rounding of each other.
"""
from __future__ import annotations

import math

import numpy as np
import torch

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85
_MASK = 0xFFFFFFFF


def philox4x32_10(ctr: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 on counters ``ctr`` (uint32 [..., 4]) with key (k0, k1)."""
    c = [ctr[..., j].astype(np.uint64) for j in range(4)]
    k0, k1 = np.uint64(key[0] & _MASK), np.uint64(key[1] & _MASK)
    m0, m1 = np.uint64(_M0), np.uint64(_M1)
    mask = np.uint64(_MASK)
    for _ in range(10):
        p0 = m0 * c[0]
        p1 = m1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & mask
        hi1, lo1 = p1 >> np.uint64(32), p1 & mask
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(_W0)) & mask
        k1 = (k1 + np.uint64(_W1)) & mask
    return np.stack(c, axis=-1).astype(np.uint32)


def uniforms(n_rows: int, vocab: int, seed: int, offset: int) -> np.ndarray:
    """U[r, i] in (0, 1) for every row and vocabulary entry (float64)."""
    nblk = (vocab + 3) // 4
    ctr = np.zeros((n_rows, nblk, 4), dtype=np.uint32)
    ctr[..., 0] = np.arange(nblk, dtype=np.uint32)[None, :]
    ctr[..., 1] = np.arange(n_rows, dtype=np.uint32)[:, None]
    ctr[..., 2] = offset & _MASK
    ctr[..., 3] = (offset >> 32) & _MASK
    w = philox4x32_10(ctr, (seed & _MASK, (seed >> 32) & _MASK)).reshape(n_rows, nblk * 4)[:, :vocab]
    return ((w >> 8).astype(np.float64) + 0.5) / 2.0 ** 24


def gumbel_scores(logits: torch.Tensor, temperature: float, seed: int, offset: int) -> np.ndarray:
    """x_i log2(e) / T - log2(-ln U_i log2(e)) per row (float64), the kernel's scores."""
    x = logits.float().double().numpy() / temperature
    n, v = x.shape
    u = uniforms(n, v, seed, offset)
    e = -np.log1p(-(1.0 - u))  # -ln U, accurate near U = 1
    return x * math.log2(math.e) - np.log2(e * math.log2(math.e))


def probs(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """softmax(logits.float() / T) in float64 (qwen3_naive.py:1413-1422)."""
    return torch.softmax(logits.double() / temperature, dim=-1)


def logprob_of(logits: torch.Tensor, tokens: torch.Tensor, temperature: float) -> torch.Tensor:
    """log_softmax(logits.float() / T)[tok] (qwen3_naive.py:1646-1650), float64."""
    lp = torch.log_softmax(logits.double() / temperature, dim=-1)
    return lp.gather(-1, tokens.long().view(-1, 1))[:, 0]


# ---------------------------------------------------------------------------
# Inverse transform sampling with one uniform per row (the fused lm_head
# sampler's draw).  Follows the same reference lines (top_k = None); the draw
# is tok = min{i : sum_{j <= i} p_j > u}, an exact sample of Categorical(p).

def uniform53(n_rows: int, seed: int, offset: int, row_counters=None) -> np.ndarray:
    """u[r] in (0, 1): words 0 and 1 of Philox4x32-10 at counter
    (0, lo32(q_r), offset_lo + hi32(q_r) mod 2^32, offset_hi), key
    (seed_lo, seed_hi), as ((w0 << 21 | w1 >> 11) + 0.5) / 2^53 (float64);
    q_r = row_counters[r] (non-negative ints), or r."""
    q = (np.arange(n_rows, dtype=np.uint64) if row_counters is None
         else np.asarray(row_counters, dtype=np.int64).astype(np.uint64))
    ctr = np.zeros((n_rows, 4), dtype=np.uint32)
    ctr[:, 1] = (q & np.uint64(_MASK)).astype(np.uint32)
    ctr[:, 2] = ((q >> np.uint64(32)) + np.uint64(offset & _MASK)) & np.uint64(_MASK)
    ctr[:, 3] = (offset >> 32) & _MASK
    w = philox4x32_10(ctr, (seed & _MASK, (seed >> 32) & _MASK))
    bits = (w[:, 0].astype(np.uint64) << np.uint64(21)) | (w[:, 1].astype(np.uint64) >> np.uint64(11))
    return (bits.astype(np.float64) + 0.5) / 2.0 ** 53


def inverse_cdf_draw(logits: torch.Tensor, temperature: float, u: np.ndarray) -> np.ndarray:
    """First index whose cumulative softmax(logits / T) probability exceeds
    u (float64), per row."""
    p = probs(logits, temperature).numpy()
    cdf = np.cumsum(p, axis=-1)
    idx = np.array([np.searchsorted(cdf[r], u[r], side="right") for r in range(p.shape[0])])
    last = np.array([np.flatnonzero(p[r] > 0)[-1] for r in range(p.shape[0])])
    return np.minimum(idx, last)


# ---------------------------------------------------------------------------
# Top-k (qwen3_naive.py:1413-1422, :1641-1650): keep the k largest of
# x = logits.float() / T, the rest -inf; softmax; draw; log_softmax at the draw.
# Ties at the k-th value keep the lowest indices.

def topk_mask(logits: torch.Tensor, k: int) -> np.ndarray:
    """Boolean [N, V]: the k kept entries of each row (value descending, then
    index ascending)."""
    x = logits.float().numpy()
    n, v = x.shape
    keep = np.zeros((n, v), dtype=bool)
    for r in range(n):
        order = np.lexsort((np.arange(v), -x[r]))   # by -x, then index
        keep[r, order[:k]] = True
    return keep


def topk_logprobs(logits: torch.Tensor, k: int, temperature: float) -> torch.Tensor:
    """log_softmax of the top-k-filtered x / T (float64; -inf off the set)."""
    keep = torch.from_numpy(topk_mask(logits, k))
    x = logits.double() / temperature
    x = x.masked_fill(~keep, float("-inf"))
    return torch.log_softmax(x, dim=-1)


def topk_inverse_cdf_draw(logits: torch.Tensor, k: int, temperature: float,
                          u: np.ndarray) -> np.ndarray:
    """First kept index (vocabulary order) whose cumulative top-k probability exceeds u."""
    p = topk_logprobs(logits, k, temperature).exp().numpy()
    cdf = np.cumsum(p, axis=-1)
    idx = np.array([np.searchsorted(cdf[r], u[r], side="right") for r in range(p.shape[0])])
    last = np.array([np.flatnonzero(p[r] > 0)[-1] for r in range(p.shape[0])])
    return np.minimum(idx, last)
