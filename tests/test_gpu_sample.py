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
