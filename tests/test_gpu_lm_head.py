"""Fused lm_head + sampling / log-prob gather (qmi_lm_head_sample,
qmi_lm_head_logprob) against the oracle on the same inputs: the logits
h . w^T computed in fp64 and rounded to bf16 (the reference's bf16 lm_head
output, qwen3_naive.py:1387 / :1607), log_softmax, and the inverse-CDF draw
(all entries, or the top k) with the same per-row Philox uniform.  Bars:
log-probs 1e-4 relative (|err| / max(|lp|, 1)); tokens equal to the oracle's
draw (a draw may differ only where u falls within fp32 rounding of a
cumulative-probability boundary, so one row in a call is allowed to differ,
and then only to a neighbouring index).  The kernel rounds an fp32 sum, the
oracle an fp64 one: where the exact logit lies within fp32 rounding of a
bf16 rounding midpoint, either neighbour is accepted."""
import numpy as np
import pytest
import torch

from oracle import sampling as OS

pytestmark = pytest.mark.gpu

LP_TOL = 1e-4


def _inputs(gpu, n, vocab, hidden=1024, w_std=0.05, seed=0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, hidden, generator=g).to(torch.bfloat16)
    w = (w_std * torch.randn(vocab, hidden, generator=g)).to(torch.bfloat16)
    return h, w, h.to(gpu), w.to(gpu)


def _logits64(h, w):
    return h.double() @ w.double().T


def _bf16(x):
    return x.float().to(torch.bfloat16).double()


def _logits_bf16(h, w):
    """(nearest, lower, upper): the fp64 logits rounded to bf16, and the
    roundings of the logits moved by the fp32 accumulation error (they differ
    from the nearest only next to a rounding midpoint)."""
    x = _logits64(h, w)
    d = 2e-6 * x.abs() + 1e-6
    return _bf16(x), _bf16(x - d), _bf16(x + d)


def _rel(a, b):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    return ((a - b).abs() / b.abs().clamp_min(1.0)).max().item()


def _assert_draws_close(tok, want):
    """Draws equal the oracle's but where u lies within the kernel / oracle
    logit rounding difference of a cumulative-probability boundary: those few
    rows move to a nearby index.  Logits whose bf16 rounding the kernel's fp32
    sum and the oracle's fp64 sum settle differently (about 1 in 1,000) shift
    the cumulative probabilities by ~1e-5 at 151,936 entries, against ~1e-3
    for a drawn token: about 1% of rows, so at most 2 or 1 in 25 are allowed."""
    diff = np.flatnonzero(tok != want)
    assert len(diff) <= max(2, len(tok) // 25), (diff, tok[diff], want[diff])
    assert (np.abs(tok[diff] - want[diff]) <= 3).all(), (diff, tok[diff], want[diff])


def _lp_err(lp, xr, lo, hi, tok, lse):
    """Per-row relative error of lp against the token's logit (either
    admissible rounding) minus lse."""
    lp = torch.as_tensor(lp, dtype=torch.float64)
    t = torch.as_tensor(tok).long()[:, None]
    errs = [((lp - (c.gather(-1, t)[:, 0] - lse)).abs() /
             (c.gather(-1, t)[:, 0] - lse).abs().clamp_min(1.0)) for c in (xr, lo, hi)]
    return torch.stack(errs).min(0).values


@pytest.mark.parametrize("n,vocab,w_std", [(1, 2085, 0.05), (37, 2085, 0.2), (64, 151936, 0.05),
                                           (100, 4096, 0.05), (130, 2085, 0.2), (300, 3000, 0.1)])
def test_lm_head_logprob_matches_oracle(pkg, gpu, n, vocab, w_std):
    h, w, hg, wg = _inputs(gpu, n, vocab, w_std=w_std, seed=n)
    g = torch.Generator().manual_seed(n + 1)
    tgt = torch.randint(0, vocab, (n,), generator=g)
    tgt[0] = vocab - 1                                     # last entry of the last tile
    print(f"[lm_head] logprob n={n} vocab={vocab}", flush=True)
    lp, lse = pkg.kernels.lm_head_logprob(hg, wg, tgt.to(gpu))
    torch.cuda.synchronize()
    xr, lo, hi = _logits_bf16(h, w)
    ref_lse = torch.logsumexp(xr, -1)
    assert _lp_err(lp.cpu(), xr, lo, hi, tgt, ref_lse).max().item() <= LP_TOL
    assert _rel(lse.cpu(), ref_lse) <= LP_TOL
    if n >= 37:
        # The bf16 rounding point is what the bar pins: the unrounded logits'
        # log-probs miss it.
        x = _logits64(h, w)
        lp_exact = x.gather(-1, tgt[:, None])[:, 0] - torch.logsumexp(x, -1)
        assert _rel(lp_exact, lp.cpu().double()) > 2 * LP_TOL


def test_lm_head_logprob_many_row_tiles(pkg, gpu):
    """Loss-step shapes (several 256-row tiles, items ordered per XCD): rows of
    a 1,100-row call match the oracle and equal, bit for bit, the same rows
    computed in a 300-row call."""
    h, w, hg, wg = _inputs(gpu, 1100, 151936, w_std=0.05, seed=17)
    tgt = torch.randint(0, 151936, (1100,), generator=torch.Generator().manual_seed(18))
    print("[lm_head] logprob 1100 rows", flush=True)
    lp, lse = pkg.kernels.lm_head_logprob(hg, wg, tgt.to(gpu))
    lp3, lse3 = pkg.kernels.lm_head_logprob(hg[:300], wg, tgt[:300].to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(lp[:300], lp3) and torch.equal(lse[:300], lse3)
    rows = torch.tensor([0, 1, 255, 256, 511, 700, 1023, 1024, 1099])
    xr, lo, hi = _logits_bf16(h[rows], w)
    ref_lse = torch.logsumexp(xr, -1)
    assert _lp_err(lp.cpu()[rows], xr, lo, hi, tgt[rows], ref_lse).max().item() <= LP_TOL
    assert _rel(lse.cpu()[rows], ref_lse) <= LP_TOL


def test_lm_head_logprob_equals_unfused_bf16_path(pkg, gpu):
    """The fused log-prob equals log_softmax over the bf16 logits of a torch
    GEMM (the autograd path: lm_head, then the log-softmax gather kernel) up to
    the logits whose rounding the two accumulation orders settle differently."""
    h, w, hg, wg = _inputs(gpu, 256, 151936, w_std=0.05, seed=3)
    tgt = torch.randint(0, 151936, (256,), generator=torch.Generator().manual_seed(4)).to(gpu)
    lp_f, _ = pkg.kernels.lm_head_logprob(hg, wg, tgt)
    logits = hg @ wg.T                                     # bf16 [256, V]
    lp_u, _ = pkg.kernels.logprob_gather(logits, tgt)
    torch.cuda.synchronize()
    d = ((lp_f - lp_u).abs() / lp_u.abs().clamp_min(1.0)).cpu()
    assert (d <= LP_TOL).float().mean().item() >= 0.97, d
    # a flipped rounding of the target's own logit moves lp by one bf16 ulp
    assert (lp_f - lp_u).abs().max().item() <= 2.0 ** -7 * 8


def test_lm_head_logprob_out_of_range_target_is_nan(pkg, gpu):
    h, w, hg, wg = _inputs(gpu, 6, 1000, w_std=0.1, seed=9)
    tgt = torch.tensor([0, -1, 999, 1000, 5, 123456], device=gpu)
    lp, lse = pkg.kernels.lm_head_logprob(hg, wg, tgt)
    torch.cuda.synchronize()
    lp = lp.cpu()
    assert torch.isnan(lp[[1, 3, 5]]).all()
    assert torch.isfinite(lp[[0, 2, 4]]).all() and torch.isfinite(lse.cpu()).all()
    xr, lo, hi = _logits_bf16(h, w)
    ok = torch.tensor([0, 2, 4])
    ref_lse = torch.logsumexp(xr, -1)
    assert _lp_err(lp[ok], xr[ok], lo[ok], hi[ok], tgt.cpu()[ok], ref_lse[ok]).max() <= LP_TOL


def test_lm_head_logprob_widest_hidden(pkg, gpu):
    """Hidden size 16,384 (the largest the C ABI takes): the log-prob row kernel
    stages the target's weight row and the hidden row (64 KB) in LDS."""
    h, w, hg, wg = _inputs(gpu, 3, 300, hidden=16384, w_std=0.01, seed=11)
    tgt = torch.tensor([0, 299, 150], device=gpu)
    lp, lse = pkg.kernels.lm_head_logprob(hg, wg, tgt)
    torch.cuda.synchronize()
    xr, lo, hi = _logits_bf16(h, w)
    ref_lse = torch.logsumexp(xr, -1)
    assert _lp_err(lp.cpu(), xr, lo, hi, tgt.cpu(), ref_lse).max().item() <= LP_TOL
    assert _rel(lse.cpu(), ref_lse) <= LP_TOL


@pytest.mark.parametrize("n,vocab,temp", [(1, 2085, 1.0), (64, 151936, 1.0), (64, 151936, 0.6),
                                          (130, 2085, 1.0), (256, 151936, 1.0), (300, 5000, 0.8)])
def test_lm_head_sample_matches_oracle(pkg, gpu, n, vocab, temp):
    h, w, hg, wg = _inputs(gpu, n, vocab, w_std=0.1, seed=7 * n + vocab)
    seed, offset = 1234 + n, 99
    print(f"[lm_head] sample n={n} vocab={vocab} T={temp}", flush=True)
    tok, lp = pkg.kernels.lm_head_sample(hg, wg, temp, seed=seed, offset=offset)
    tok2, _ = pkg.kernels.lm_head_sample(hg, wg, temp, seed=seed, offset=offset)
    torch.cuda.synchronize()
    tok, lp = tok.cpu(), lp.cpu()
    assert torch.equal(tok, tok2.cpu())                       # reproducible
    xr, lo, hi = _logits_bf16(h, w)
    u = OS.uniform53(n, seed, offset)
    want = OS.inverse_cdf_draw(xr, temp, u)
    _assert_draws_close(tok.numpy(), want)
    lse = torch.logsumexp(xr / temp, -1)
    assert _lp_err(lp, xr / temp, lo / temp, hi / temp, tok, lse).max().item() <= LP_TOL


def _topk_case(kind, n, vocab, seed):
    """Hidden states and weights for the fused top-k tests.
    plain:     random;
    clustered: the 40 largest logits of every row in tile 0 (entries 0-39),
               so tile 0 saturates and is recomputed in full;
    ties16:    16 distinct weight rows repeated, every tile holding 8 copies
               of each row's maximum: ties at the k-th value across tiles."""
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, 1024, generator=g)
    if kind == "plain":
        w = 0.1 * torch.randn(vocab, 1024, generator=g)
    elif kind == "clustered":
        h = h[:1].expand(n, -1) + 0.01 * torch.randn(n, 1024, generator=g)
        w = 0.05 * torch.randn(vocab, 1024, generator=g)
        c = torch.linspace(3.0, 1.0, 40)[:, None]
        w[:40] = c * h[0] / h[0].norm() * 2 + 0.01 * torch.randn(40, 1024, generator=g)
    else:
        base = 0.1 * torch.randn(16, 1024, generator=g)
        w = base[torch.arange(vocab) % 16]
    return h.to(torch.bfloat16), w.to(torch.bfloat16)


@pytest.mark.parametrize("kind,n,vocab,k,temp", [
    ("plain", 1, 2085, 20, 1.0), ("plain", 64, 151936, 20, 0.6), ("plain", 256, 151936, 20, 1.0),
    ("plain", 100, 4096, 64, 0.8), ("plain", 37, 3000, 1, 1.0), ("plain", 70, 300, 64, 1.0),
    ("plain", 300, 2085, 20, 0.8),
    ("clustered", 8, 151936, 20, 1.0), ("clustered", 80, 5000, 32, 0.7),
    ("clustered", 260, 3000, 20, 1.0),
    ("ties16", 4, 4096, 20, 1.0), ("ties16", 90, 4096, 37, 0.9)])
def test_lm_head_topk_matches_oracle(pkg, gpu, kind, n, vocab, k, temp):
    """Fused lm_head + top-k sampling (the reference default k = 20) against
    the oracle over the bf16 logits: the drawn token is in the kept set (ties at
    the k-th value keep the lowest indices), equals the oracle's inverse-CDF
    draw for the same uniform, and its log-probability under the top-k
    distribution is within 1e-4."""
    h, w = _topk_case(kind, n, vocab, seed=n * 13 + k)
    hg, wg = h.to(gpu), w.to(gpu)
    seed, offset = 500 + n, 3
    print(f"[lm_head] topk {kind} n={n} vocab={vocab} k={k} T={temp}", flush=True)
    tok, lp = pkg.kernels.lm_head_sample(hg, wg, temp, seed=seed, offset=offset, top_k=k)
    torch.cuda.synchronize()
    tok, lp = tok.cpu(), lp.cpu()
    xr, lo, hi = _logits_bf16(h, w)
    amb = (lo != hi).any(-1).numpy()           # rows with a logit next to a midpoint
    keep = OS.topk_mask(xr, k)
    inset = keep[np.arange(n), tok.numpy()]
    assert (inset | amb).all()
    want = OS.topk_inverse_cdf_draw(xr, k, temp, OS.uniform53(n, seed, offset))
    bad = np.flatnonzero((tok.numpy() != want) & ~amb)
    assert len(bad) <= max(1, n // 100), (bad, tok.numpy()[bad], want[bad])
    ref = OS.topk_logprobs(xr, k, temp).gather(-1, tok[:, None])[:, 0]
    err = ((lp.double() - ref).abs() / ref.abs().clamp_min(1.0)).numpy()
    assert (err[~amb & inset] <= LP_TOL).all(), err.max()
    if k == 1:
        assert (lp == 0).all()


def test_lm_head_topk_frequencies(pkg, gpu):
    """4,000 rows with one hidden state, k = 5: the draws follow the top-5
    softmax (chi-square) and never leave the kept set."""
    h, w, hg, wg = _inputs(gpu, 1, 700, w_std=0.15, seed=21)
    n = 4000
    toks = pkg.kernels.lm_head_sample(hg.expand(n, -1).contiguous(), wg, 0.8, seed=5,
                                      top_k=5)[0].cpu().numpy()
    xr, _, _ = _logits_bf16(h, w)
    p = OS.topk_logprobs(xr, 5, 0.8)[0].exp().numpy()
    counts = np.bincount(toks, minlength=700)
    assert counts[p == 0].sum() == 0
    from scipy import stats
    kept = p > 0
    chi2 = ((counts[kept] - n * p[kept]) ** 2 / (n * p[kept])).sum()
    assert chi2 < stats.chi2.ppf(0.999, df=kept.sum() - 1), chi2


@pytest.mark.parametrize("top_k", [None, 20])
def test_lm_head_row_counters_make_rows_batch_independent(pkg, gpu, top_k):
    """With per-row counters a row's draw depends on (seed, offset, its counter)
    and its hidden state only: a permuted batch gives the permuted tokens, and
    each token equals the oracle's draw with that row's uniform."""
    h, w, hg, wg = _inputs(gpu, 96, 151936, w_std=0.1, seed=31)
    q = torch.tensor([(j % 7 << 32) | (1000 + j) for j in range(96)], dtype=torch.int64)
    perm = torch.randperm(96, generator=torch.Generator().manual_seed(2))
    t1, l1 = pkg.kernels.lm_head_sample(hg, wg, 1.0, seed=77, offset=4, top_k=top_k,
                                        row_counters=q.to(gpu))
    t2, l2 = pkg.kernels.lm_head_sample(hg[perm.to(gpu)], wg, 1.0, seed=77, offset=4, top_k=top_k,
                                        row_counters=q[perm].to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(t1.cpu()[perm], t2.cpu()) and torch.equal(l1.cpu()[perm], l2.cpu())
    xr, _, _ = _logits_bf16(h, w)
    u = OS.uniform53(96, 77, 4, q.numpy())
    want = (OS.inverse_cdf_draw(xr, 1.0, u) if top_k is None
            else OS.topk_inverse_cdf_draw(xr, top_k, 1.0, u))
    _assert_draws_close(t1.cpu().numpy(), want)


def test_lm_head_topk_rejects_large_k(pkg, gpu):
    h, w, hg, wg = _inputs(gpu, 2, 1000, seed=1)
    with pytest.raises(ValueError):
        pkg.kernels.lm_head_sample(hg, wg, 1.0, top_k=65)
    st = pkg._lib.lib().qmi_lm_head_sample(hg.data_ptr(), 1024, 2, wg.data_ptr(), 1024, 1000, 1024,
                                           1.0, 65, 1, 0, None, hg.data_ptr(), None, hg.data_ptr(),
                                           1 << 20, None)
    assert st == -4


def test_lm_head_sample_frequencies(pkg, gpu):
    """2,000 rows with the same hidden state: the token frequencies follow
    softmax(x / T) (chi-square over the entries with expected count >= 20)."""
    h, w, hg, wg = _inputs(gpu, 1, 1000, w_std=0.15, seed=3)
    n = 2000
    toks = pkg.kernels.lm_head_sample(hg.expand(n, -1).contiguous(), wg, 0.9, seed=77)[0].cpu()
    p = OS.probs(_logits_bf16(h, w)[0], 0.9)[0].numpy()
    counts = np.bincount(toks.numpy(), minlength=1000)
    keep = n * p >= 20
    from scipy import stats
    obs = np.append(counts[keep], counts[~keep].sum())
    exp = np.append(n * p[keep], n * p[~keep].sum())
    chi2 = ((obs - exp) ** 2 / exp).sum()
    assert chi2 < stats.chi2.ppf(0.999, df=len(obs) - 1), chi2


def test_lm_head_under_graph_capture(pkg, gpu):
    """Capturable: a graph replay gives the eager tokens and log-probs."""
    h, w, hg, wg = _inputs(gpu, 48, 3000, w_std=0.1, seed=5)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.kernels.lm_head_sample(hg, wg, 1.0, seed=5, offset=1)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tok_g, lp_g = pkg.kernels.lm_head_sample(hg, wg, 1.0, seed=5, offset=1)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        tok_e, lp_e = pkg.kernels.lm_head_sample(hg, wg, 1.0, seed=5, offset=1)
        torch.cuda.synchronize()
        assert torch.equal(tok_g, tok_e) and torch.equal(lp_g, lp_e)


@pytest.mark.parametrize("reduction", ["token", "seq"])
def test_grpo_loss_from_hidden_matches_oracle(pkg, gpu, reduction):
    """The loss step from final hidden states (fused lm_head log-probs, shifted
    alignment, advantages, clipped loss) against the oracle on fp64 logits."""
    from oracle import grpo as OG
    g = torch.Generator().manual_seed(11)
    b, t, v = 8, 40, 3000
    h = torch.randn(b, t, 1024, generator=g).to(torch.bfloat16)
    w = (0.08 * torch.randn(v, 1024, generator=g)).to(torch.bfloat16)
    ids = torch.randint(0, v, (b, t), generator=g)
    lens = torch.tensor([10, 39, 25, 3, 39, 17, 30, 1])
    mask = (torch.arange(t)[None] >= 1) & (torch.arange(t)[None] <= lens[:, None])
    mask = mask.float()
    x = _bf16(h.double() @ w.double().T)[:, :-1]
    lp_ref = torch.log_softmax(x, -1).gather(-1, ids[:, 1:, None])[..., 0]
    old = torch.zeros(b, t)
    old[:, 1:] = (lp_ref + 0.3 * torch.randn(b, t - 1, generator=g, dtype=torch.float64)).float()
    rewards = torch.tensor([1.0, 0.0, 1.0, 1.0, 0.0, 0.0, 1.0, 0.0])
    pids = torch.tensor([0, 0, 0, 0, 1, 1, 1, 1])
    print(f"[lm_head] grpo loss from hidden ({reduction})", flush=True)
    loss, lp, adv = pkg.grpo_loss_from_hidden(h.to(gpu), w.to(gpu), ids.to(gpu), old.to(gpu),
                                              mask.to(gpu), rewards.to(gpu), pids.to(gpu), 1e-4,
                                              0.2, reduction, shift=True)
    torch.cuda.synchronize()
    adv_ref = OG.advantage(rewards.double(), pids, 1e-4)
    m = mask[:, 1:].double()
    loss_ref = OG.ppo_loss(old[:, 1:].double(), lp_ref, adv_ref[:, None] * m, m, 0.2, reduction)
    # (logits within fp32 rounding of a bf16 midpoint may round either way)
    d = ((lp.cpu().double() - lp_ref).abs() / lp_ref.abs().clamp_min(1.0))
    xx = (h.double() @ w.double().T)[:, :-1]
    amb = (_bf16(xx - 2e-6 * xx.abs() - 1e-6) != _bf16(xx + 2e-6 * xx.abs() + 1e-6)).any(-1)
    assert (d[~amb] <= LP_TOL).all() and (d <= 2.0 ** -6).all()
    assert _rel(adv.cpu(), adv_ref) <= LP_TOL
    if not amb.any():
        assert abs(loss.item() - loss_ref.item()) <= LP_TOL * max(1.0, abs(loss_ref.item()))


def test_forward_logprob_without_grad_is_fused(pkg, gpu):
    """forward_logprob under no_grad runs the fused lm_head kernel: against the
    fp64 log-softmax of the model's own final hidden states at the unshifted
    tokens (qwen3_grpo_train.py:46-53)."""
    cfg = pkg.Qwen3Config(num_hidden_layers=2, vocab_size=2048, tie_word_embeddings=False)
    torch.manual_seed(0)
    m = pkg.Qwen3ForCausalLM(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            else:
                p.normal_(0, 0.05)
    m = m.to(gpu).to(torch.bfloat16)
    ids = torch.randint(0, 2048, (3, 50), generator=torch.Generator().manual_seed(1)).to(gpu)
    with torch.no_grad():
        lp = pkg.forward_logprob(m, ids)
        hid = m.model(ids)
    torch.cuda.synchronize()
    hc, wc = hid.cpu().reshape(-1, 1024), m.lm_head.weight.cpu()
    xr, lo, hi = _logits_bf16(hc, wc)
    lse = torch.logsumexp(xr, -1)
    assert lp.shape == ids.shape
    assert _lp_err(lp.cpu().reshape(-1), xr, lo, hi, ids.cpu().reshape(-1), lse).max() <= LP_TOL


# Shapes at the kernels' edges: vocabularies below one 32-entry slice or one
# 128-entry tile, or one entry past them; hidden sizes of one 64-wide chunk, three
# chunks and 2,048; the row counts on both sides of each configuration change
# (64 / 65, 256 / 257); top-1 and top-64.
EDGE_CASES = [  # (rows, vocab, hidden, top_k, temperature)
    (1, 7, 64, None, 1.0),
    (3, 33, 64, None, 0.7),
    (5, 129, 128, 1, 1.0),
    (64, 200, 2048, None, 1.0),
    (65, 200, 2048, 20, 1.0),
    (256, 1000, 192, None, 1.3),
    (257, 1000, 192, 64, 1.0),
    (511, 131, 64, 20, 0.9),
]


@pytest.mark.parametrize("n,vocab,hidden,k,temp", EDGE_CASES)
def test_lm_head_edge_shapes(pkg, gpu, n, vocab, hidden, k, temp):
    """Sampling (all entries or top k) and the target log-prob at edge shapes,
    against the oracle with the bars above."""
    h, w, hg, wg = _inputs(gpu, n, vocab, hidden=hidden, w_std=0.3 / hidden ** 0.5 * 8,
                           seed=n + vocab + hidden)
    seed, offset = 900 + n, 11
    print(f"[lm_head] edge n={n} vocab={vocab} hidden={hidden} k={k} T={temp}", flush=True)
    tok, lp = pkg.kernels.lm_head_sample(hg, wg, temp, seed=seed, offset=offset, top_k=k)
    tgt = torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(n))
    tgt[0] = vocab - 1
    lpt, lse = pkg.kernels.lm_head_logprob(hg, wg, tgt.to(gpu))
    torch.cuda.synchronize()
    tok, lp, lpt, lse = tok.cpu(), lp.cpu(), lpt.cpu(), lse.cpu()
    xr, lo, hi = _logits_bf16(h, w)
    u = OS.uniform53(n, seed, offset)
    assert ((tok >= 0) & (tok < vocab)).all()
    if k is None or k >= vocab:
        _assert_draws_close(tok.numpy(), OS.inverse_cdf_draw(xr, temp, u))
        ref_lse = torch.logsumexp(xr / temp, -1)
        assert _lp_err(lp, xr / temp, lo / temp, hi / temp, tok, ref_lse).max().item() <= LP_TOL
    else:
        amb = (lo != hi).any(-1).numpy()
        keep = OS.topk_mask(xr, k)
        inset = keep[np.arange(n), tok.numpy()]
        assert (inset | amb).all()
        want = OS.topk_inverse_cdf_draw(xr, k, temp, u)
        bad = np.flatnonzero((tok.numpy() != want) & ~amb)
        assert len(bad) <= max(1, n // 100), (bad, tok.numpy()[bad], want[bad])
        ref = OS.topk_logprobs(xr, k, temp).gather(-1, tok[:, None])[:, 0]
        err = ((lp.double() - ref).abs() / ref.abs().clamp_min(1.0)).numpy()
        assert (err[~amb & inset] <= LP_TOL).all(), err.max()
    ref_lse = torch.logsumexp(xr, -1)
    assert _lp_err(lpt, xr, lo, hi, tgt, ref_lse).max().item() <= LP_TOL
    assert _rel(lse, ref_lse) <= LP_TOL
