"""Sampling oracle: Philox4x32-10 against its authors' known-answer vectors,
the uniform mapping, and the Gumbel-max draw against softmax frequencies."""
import numpy as np
import torch
from scipy import stats

from oracle import sampling as OS


def test_philox_known_answers():
    # Known-answer vectors of Philox4x32-10 published with the Random123
    # library (counter, key) -> output.
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in cases:
        got = OS.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
        assert tuple(int(x) for x in got) == want


def test_uniforms_open_interval_and_layout():
    u = OS.uniforms(3, 11, seed=5, offset=7)
    assert u.shape == (3, 11) and (u > 0).all() and (u < 1).all()
    # element i of row r is word i % 4 of block (i // 4, r, offset)
    w = OS.philox4x32_10(np.array([[2, 1, 7, 0]], dtype=np.uint32), (5, 0))[0]
    assert u[1, 9] == ((int(w[1]) >> 8) + 0.5) / 2 ** 24


def test_gumbel_max_matches_softmax_frequencies():
    logits = torch.tensor([[2.0, 1.0, 0.5, 0.0, -1.0, 3.0]]).to(torch.bfloat16)
    for temp in (1.0, 0.7):
        n = 40000
        sc = OS.gumbel_scores(logits.expand(n, -1).contiguous(), temp, seed=11, offset=3)
        counts = np.bincount(sc.argmax(-1), minlength=6)
        p = OS.probs(logits, temp)[0].numpy()
        chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
        assert chi2 < stats.chi2.ppf(0.999, df=5), (temp, chi2, counts, n * p)


def test_logprob_of_is_log_softmax():
    g = torch.Generator().manual_seed(0)
    logits = (3 * torch.randn(4, 50, generator=g)).to(torch.bfloat16)
    tok = torch.tensor([0, 7, 49, 3])
    lp = OS.logprob_of(logits, tok, 0.8)
    x = logits.double() / 0.8
    want = x.gather(-1, tok[:, None])[:, 0] - torch.logsumexp(x, -1)
    assert torch.allclose(lp, want, atol=1e-12)
    # probabilities of a row sum to one
    assert torch.allclose(OS.probs(logits, 0.8).sum(-1), torch.ones(4, dtype=torch.float64))


def test_uniform53_layout_and_range():
    u = OS.uniform53(5, seed=(9 << 32) | 5, offset=(3 << 32) | 7)
    assert u.shape == (5,) and (u > 0).all() and (u < 1).all()
    w = OS.philox4x32_10(np.array([[0, 3, 7, 3]], dtype=np.uint32), (5, 9))[0]
    want = (((int(w[0]) << 21) | (int(w[1]) >> 11)) + 0.5) / 2 ** 53
    assert u[3] == want
    assert len(set(u.tolist())) == 5


def test_uniform53_row_counters():
    """Row counter q occupies counter words 1-2: q = r reproduces the default
    layout, and q = (j << 32) | s is row s's block of a call at offset + j."""
    seed, off = (7 << 32) | 3, (2 << 32) | 11
    assert (OS.uniform53(6, seed, off, np.arange(6)) == OS.uniform53(6, seed, off)).all()
    q = [(5 << 32) | 4, (0 << 32) | 1, (9 << 32) | 0]
    got = OS.uniform53(3, seed, off, q)
    assert got[0] == OS.uniform53(5, seed, off + 5)[4]
    assert got[1] == OS.uniform53(2, seed, off)[1]
    assert got[2] == OS.uniform53(1, seed, off + 9)[0]
    # the low word of the offset wraps into nothing: (offset_lo + hi32(q)) mod 2^32
    w = OS.philox4x32_10(np.array([[0, 4, (0xFFFFFFFF + 5) & 0xFFFFFFFF, 0]], dtype=np.uint32),
                         (3, 7))[0]
    want = (((int(w[0]) << 21) | (int(w[1]) >> 11)) + 0.5) / 2 ** 53
    assert OS.uniform53(1, seed, 0xFFFFFFFF, [(5 << 32) | 4])[0] == want


def test_inverse_cdf_closed_forms():
    # p = softmax([0, 0]) = (1/2, 1/2): u below 1/2 draws 0, above draws 1.
    x = torch.zeros(2, 2)
    assert OS.inverse_cdf_draw(x, 1.0, np.array([0.25, 0.75])).tolist() == [0, 1]
    # p = (1/6, 2/6, 3/6): boundaries at 1/6 and 1/2.
    x = torch.log(torch.tensor([[1.0, 2.0, 3.0]])).expand(4, -1)
    got = OS.inverse_cdf_draw(x, 1.0, np.array([0.1, 0.2, 0.49, 0.51]))
    assert got.tolist() == [0, 1, 1, 2]
    # Entries of zero probability are never drawn, even for u next to 1.
    x = torch.tensor([[0.0, 1.0, float("-inf")]])
    assert OS.inverse_cdf_draw(x, 1.0, np.array([1 - 2 ** -53])).tolist() == [1]


def test_inverse_cdf_matches_softmax_frequencies():
    logits = torch.tensor([[2.0, 1.0, 0.5, 0.0, -1.0, 3.0]]).to(torch.bfloat16)
    n = 40000
    for temp in (1.0, 0.7):
        u = OS.uniform53(n, seed=13, offset=5)
        tok = OS.inverse_cdf_draw(logits.expand(n, -1).contiguous(), temp, u)
        counts = np.bincount(tok, minlength=6)
        p = OS.probs(logits, temp)[0].numpy()
        chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
        assert chi2 < stats.chi2.ppf(0.999, df=5), (temp, chi2, counts, n * p)


def test_topk_set_matches_torch_topk_without_ties():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, 500, generator=g, dtype=torch.float64).float()   # distinct values
    keep = OS.topk_mask(x, 20)
    want = torch.zeros_like(x, dtype=torch.bool).scatter(-1, torch.topk(x, 20).indices, True)
    assert (keep == want.numpy()).all() and keep.sum(1).tolist() == [20] * 6


def test_topk_ties_keep_lowest_indices_and_closed_forms():
    x = torch.tensor([[1.0, 3.0, 2.0, 3.0, 2.0, 2.0, 0.0]])
    assert np.flatnonzero(OS.topk_mask(x, 3)[0]).tolist() == [1, 2, 3]   # 3, 3 then the first 2
    # k = 1 always draws the (first) maximum, with log-prob 0.
    assert OS.topk_inverse_cdf_draw(x, 1, 0.7, np.array([0.999])).tolist() == [1]
    assert OS.topk_logprobs(x, 1, 0.7)[0, 1].item() == 0.0
    # k = V is plain sampling.
    u = np.array([0.3])
    assert OS.topk_inverse_cdf_draw(x, 7, 1.0, u).tolist() == OS.inverse_cdf_draw(x, 1.0, u).tolist()
    # Two kept entries of logits 3 and 3 - ln 3: probabilities 3/4 and 1/4.
    y = torch.tensor([[3.0, 3.0 - float(np.log(3.0)), -5.0]])
    lp = OS.topk_logprobs(y, 2, 1.0)[0]
    # (the logits are fp32: 3 - ln 3 carries one fp32 rounding)
    assert abs(lp[0].item() - np.log(0.75)) < 1e-7 and abs(lp[1].item() - np.log(0.25)) < 1e-7
    assert OS.topk_inverse_cdf_draw(y.expand(2, -1), 2, 1.0, np.array([0.74, 0.76])).tolist() == [0, 1]


def test_topk_draw_frequencies():
    logits = torch.tensor([[2.0, 1.0, 0.5, 0.0, -1.0, 3.0, 2.5, -0.5]]).to(torch.bfloat16)
    n = 40000
    u = OS.uniform53(n, seed=21, offset=9)
    tok = OS.topk_inverse_cdf_draw(logits.expand(n, -1).contiguous(), 4, 0.8, u)
    p = OS.topk_logprobs(logits, 4, 0.8)[0].exp().numpy()
    counts = np.bincount(tok, minlength=8)
    assert counts[p == 0].sum() == 0
    kept = p > 0
    chi2 = ((counts[kept] - n * p[kept]) ** 2 / (n * p[kept])).sum()
    assert chi2 < stats.chi2.ppf(0.999, df=kept.sum() - 1)
