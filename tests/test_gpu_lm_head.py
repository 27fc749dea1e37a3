"""Fused lm_head + sampling / log-prob gather (qmi_lm_head_sample,
qmi_lm_head_logprob) against the oracle on the same inputs: fp64 logits
h . w^T, log_softmax, and the inverse-CDF draw with the same per-row Philox
uniform.  Bars: log-probs 1e-4 relative (|err| / max(|lp|, 1)); tokens equal
to the oracle's draw (a draw may differ only where u falls within fp32
rounding of a cumulative-probability boundary, so one row in a call is
allowed to differ, and then only to a neighbouring index)."""
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


def _rel(a, b):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    return ((a - b).abs() / b.abs().clamp_min(1.0)).max().item()


@pytest.mark.parametrize("n,vocab,w_std", [(1, 2085, 0.05), (37, 2085, 0.2), (64, 151936, 0.05),
                                           (100, 4096, 0.05), (300, 3000, 0.1)])
def test_lm_head_logprob_matches_oracle(pkg, gpu, n, vocab, w_std):
    h, w, hg, wg = _inputs(gpu, n, vocab, w_std=w_std, seed=n)
    g = torch.Generator().manual_seed(n + 1)
    tgt = torch.randint(0, vocab, (n,), generator=g)
    tgt[0] = vocab - 1                                     # last entry of the last tile
    print(f"[lm_head] logprob n={n} vocab={vocab}", flush=True)
    lp, lse = pkg.kernels.lm_head_logprob(hg, wg, tgt.to(gpu))
    torch.cuda.synchronize()
    x = _logits64(h, w)
    ref_lse = torch.logsumexp(x, -1)
    ref_lp = x.gather(-1, tgt[:, None])[:, 0] - ref_lse
    assert _rel(lp.cpu(), ref_lp) <= LP_TOL
    assert _rel(lse.cpu(), ref_lse) <= LP_TOL


@pytest.mark.parametrize("n,vocab,temp", [(1, 2085, 1.0), (64, 151936, 1.0), (64, 151936, 0.6),
                                          (256, 151936, 1.0), (300, 5000, 0.8)])
def test_lm_head_sample_matches_oracle(pkg, gpu, n, vocab, temp):
    h, w, hg, wg = _inputs(gpu, n, vocab, w_std=0.1, seed=7 * n + vocab)
    seed, offset = 1234 + n, 99
    print(f"[lm_head] sample n={n} vocab={vocab} T={temp}", flush=True)
    tok, lp = pkg.kernels.lm_head_sample(hg, wg, temp, seed=seed, offset=offset)
    tok2, _ = pkg.kernels.lm_head_sample(hg, wg, temp, seed=seed, offset=offset)
    torch.cuda.synchronize()
    tok, lp = tok.cpu(), lp.cpu()
    assert torch.equal(tok, tok2.cpu())                       # reproducible
    x = _logits64(h, w)
    u = OS.uniform53(n, seed, offset)
    want = OS.inverse_cdf_draw(x, temp, u)
    diff = np.flatnonzero(tok.numpy() != want)
    assert len(diff) <= 1, (diff, tok.numpy()[diff], want[diff])
    for r in diff:
        assert abs(int(tok[r]) - int(want[r])) == 1
    ref_lp = OS.logprob_of(x, tok, temp)
    assert _rel(lp, ref_lp) <= LP_TOL


def test_lm_head_sample_frequencies(pkg, gpu):
    """2,000 rows with the same hidden state: the token frequencies follow
    softmax(x / T) (chi-square over the entries with expected count >= 20)."""
    h, w, hg, wg = _inputs(gpu, 1, 1000, w_std=0.15, seed=3)
    n = 2000
    toks = pkg.kernels.lm_head_sample(hg.expand(n, -1).contiguous(), wg, 0.9, seed=77)[0].cpu()
    p = OS.probs(_logits64(h, w), 0.9)[0].numpy()
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
    x = (h.double() @ w.double().T)[:, :-1]
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
    assert _rel(lp.cpu(), lp_ref) <= LP_TOL
    assert _rel(adv.cpu(), adv_ref) <= LP_TOL
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
    x = hid.double().cpu() @ m.lm_head.weight.double().cpu().T
    ref = torch.log_softmax(x, -1).gather(-1, ids.cpu()[..., None])[..., 0]
    assert lp.shape == ids.shape
    assert _rel(lp.cpu(), ref) <= LP_TOL
