"""Fused sampler (qmi_sample_tokens) against the sampling oracle.

* The oracle follows the same Philox4x32-10 / Gumbel-max stream in float64,
  so wherever its top two scores are more than 1e-3 (log2 units) apart the
  kernel must draw exactly the oracle's token.
* Drawn log-probabilities: 1e-4 relative (|err| / max(|ref|, 1)) against
  log_softmax(logits.float() / T).
* Frequencies: chi-square against softmax(logits / T) at p = 0.001.
"""
import numpy as np
import pytest
import torch
from scipy import stats

from oracle import sampling as OS

pytestmark = pytest.mark.gpu


def _logits(seed, n, v, std=3.0):
    g = torch.Generator().manual_seed(seed)
    return (std * torch.randn(n, v, generator=g)).to(torch.bfloat16)


def _agree(pkg, gpu, logits_cpu, logits_gpu, temp, seed, offset):
    tok, lp = pkg.kernels.sample_tokens(logits_gpu, temp, seed=seed, offset=offset)
    torch.cuda.synchronize()
    tok, lp = tok.cpu(), lp.cpu()
    sc = OS.gumbel_scores(logits_cpu, temp, seed, offset)
    top2 = np.sort(sc, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-3
    want = sc.argmax(-1)
    assert clear.mean() > 0.9
    assert (tok.numpy()[clear] == want[clear]).all()
    ref_lp = OS.logprob_of(logits_cpu, tok, temp)
    err = ((lp.double() - ref_lp).abs() / ref_lp.abs().clamp_min(1.0)).max().item()
    assert err <= 1e-4, err
    return tok


@pytest.mark.parametrize("v,temp", [(4096, 1.0), (1003, 0.7), (151936, 1.0), (64, 2.0)])
def test_sample_matches_oracle_stream(pkg, gpu, v, temp):
    n = 8 if v > 100000 else 96
    lg = _logits(v, n, v)
    print(f"[sample] v={v} T={temp}", flush=True)
    _agree(pkg, gpu, lg, lg.to(gpu), temp, seed=1234 + v, offset=5)


@pytest.mark.parametrize("width", [1000, 1001])
def test_sample_strided_rows(pkg, gpu, width):
    """Rows of a wider buffer: vector path with (1001) and without (1000) a tail."""
    full = _logits(7, 40, 1024)
    lg = full[:, :width]
    print(f"[sample] strided width={width}", flush=True)
    _agree(pkg, gpu, lg.contiguous(), full.to(gpu)[:, :width], 1.0, seed=99, offset=0)


@pytest.mark.parametrize("temp", [1.0, 0.5])
def test_sample_frequencies_match_softmax(pkg, gpu, temp):
    base = torch.tensor([[2.0, 1.0, 0.5, 0.0, -1.0, 3.0, -2.0, 1.5]]).to(torch.bfloat16)
    n = 100000
    print(f"[sample] frequencies T={temp}", flush=True)
    tok, _ = pkg.kernels.sample_tokens(base.expand(n, -1).contiguous().to(gpu), temp, seed=3)
    counts = np.bincount(tok.cpu().numpy(), minlength=8)
    p = OS.probs(base, temp)[0].numpy()
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < stats.chi2.ppf(0.999, df=7), (chi2, counts, n * p)


def test_sample_dominant_token_and_determinism(pkg, gpu):
    lg = _logits(11, 32, 2048, std=1.0)
    lg[:, 777] = 60.0  # p(777) ~ 1 - 1e-22
    g = lg.to(gpu)
    print("[sample] dominant + determinism", flush=True)
    tok, lp = pkg.kernels.sample_tokens(g, 1.0, seed=1, offset=0)
    assert (tok.cpu() == 777).all() and lp.abs().max().item() < 1e-5
    flat = _logits(12, 64, 4096, std=0.1).to(gpu)
    a, _ = pkg.kernels.sample_tokens(flat, 1.0, seed=8, offset=0)
    b, _ = pkg.kernels.sample_tokens(flat, 1.0, seed=8, offset=0)
    c, _ = pkg.kernels.sample_tokens(flat, 1.0, seed=8, offset=1)
    assert torch.equal(a, b) and (a != c).float().mean().item() > 0.9


def test_sample_rejects_bad_arguments(pkg, gpu):
    lg = _logits(13, 4, 64).to(gpu)
    for t in (0.0, -1.0, float("inf")):
        with pytest.raises(ValueError):
            pkg.kernels.sample_tokens(lg, t)
    with pytest.raises(ValueError):
        pkg.kernels.sample_tokens(lg.float(), 1.0)


@pytest.mark.parametrize("n,vocab,k,temp", [(1, 1000, 1, 1.0), (8, 1000, 20, 0.6),
                                            (64, 151936, 20, 0.6), (256, 151936, 20, 1.0),
                                            (16, 5000, 1000, 1.0), (5, 40, 40, 0.9)])
def test_topk_sampler_matches_oracle(pkg, gpu, n, vocab, k, temp):
    """Top-k sampling (the reference's default k = 20) against the oracle: the
    same kept set (ties at the k-th value keep the lowest indices), the same
    inverse-CDF draw for the same per-row uniform, log-probs to 1e-4."""
    g = torch.Generator().manual_seed(n * 31 + k)
    # bf16 logits of std 3: many ties at the k-th value across 151,936 entries.
    logits = (3 * torch.randn(n, vocab, generator=g)).to(torch.bfloat16)
    seed, offset = 99 + n, 5
    print(f"[topk] n={n} vocab={vocab} k={k} T={temp}", flush=True)
    tok, lp = pkg.kernels.sample_tokens_topk(logits.to(gpu), k, temp, seed=seed, offset=offset)
    torch.cuda.synchronize()
    tok, lp = tok.cpu(), lp.cpu()
    keep = OS.topk_mask(logits, k)
    assert keep[np.arange(n), tok.numpy()].all()
    want = OS.topk_inverse_cdf_draw(logits, k, temp, OS.uniform53(n, seed, offset))
    assert (tok.numpy() == want).mean() >= 0.99, (tok.numpy(), want)
    ref = OS.topk_logprobs(logits, k, temp).gather(-1, tok[:, None])[:, 0]
    assert ((lp.double() - ref).abs() / ref.abs().clamp_min(1.0)).max().item() <= 1e-4


def test_topk_engine_path(pkg, gpu):
    """generate_continuous with the reference's default top_k = 20 runs the HIP
    top-k sampler: every generated token is among the most likely under the
    model's own logits at that position (the batch forward's bf16 logits may
    order the entries near the 20th slightly differently, hence 24)."""
    cfg = pkg.Qwen3Config(num_hidden_layers=2, vocab_size=2048, tie_word_embeddings=False)
    torch.manual_seed(0)
    m = pkg.Qwen3ForCausalLM(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.fill_(1.0)
            else:
                p.normal_(0, 0.1)
    m = m.to(gpu).to(torch.bfloat16).eval()
    m.allocate_global_kv_cache(num_blocks=16)
    prompts = [torch.randint(0, 2048, (1, 30), generator=torch.Generator().manual_seed(2))]
    toks, gen, lps, _ = m.generate_continuous_with_logprobs(prompts, max_new_tokens=8,
                                                            temperature=0.7, top_k=20)
    seq = torch.tensor(toks[0], device=gpu)[None]
    with torch.no_grad():
        logits = m(seq)[0].float()
    for j, t in enumerate(gen[0]):
        row = logits[30 + j - 1]
        assert t in torch.topk(row, 24).indices.tolist()
        lp_ref = torch.log_softmax(torch.topk(row / 0.7, 20).values, -1)
        assert lps[0][j] <= 0.0 and lps[0][j] >= lp_ref.min().item() - 0.1
