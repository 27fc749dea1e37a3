"""GRPO loss-step parity against the oracle.

Tolerance: logprobs and loss within 1e-4 relative error in fp32, measured as
|err| / max(|ref|, 1) so near-zero log-probabilities are not ill-conditioned.
"""
import math

import pytest
import torch

from oracle import grpo as OG
from oracle import workloads as W

pytestmark = pytest.mark.gpu

RTOL = 1e-4


def rel_err(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).abs() / b.abs().clamp_min(1.0)).max().item()


def _small_case(seed, n_seq=8, n_tok=16, vocab=1024, group=4):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(n_seq, n_tok, vocab, generator=g) * 2).to(torch.bfloat16)
    ids = torch.randint(0, vocab, (n_seq, n_tok), generator=g)
    lens = torch.randint(1, n_tok + 1, (n_seq,), generator=g)
    mask = (torch.arange(n_tok)[None] < lens[:, None]).float()
    new, _ = OG.logprob_gather(logits, ids)
    old = new + 0.3 * torch.randn(n_seq, n_tok, generator=g)
    rewards = torch.bernoulli(torch.full((n_seq,), 0.5), generator=g)
    rewards[0], rewards[1] = 1.0, 0.0  # every group of the first prompt has both values
    pids = torch.arange(n_seq // group).repeat_interleave(group)
    return dict(logits=logits, ids=ids, mask=mask, old=old, rewards=rewards, pids=pids)


@pytest.mark.parametrize("vocab", [1024, 1001, 151936])
def test_logprob_gather_matches_oracle(pkg, gpu, vocab):
    c = _small_case(1, n_seq=3, n_tok=5, vocab=vocab)
    print(f"[grpo] logprob vocab={vocab}", flush=True)
    lp, lse = pkg.kernels.logprob_gather(c["logits"].to(gpu), c["ids"].to(gpu))
    torch.cuda.synchronize()
    rlp, rlse = OG.logprob_gather(c["logits"], c["ids"])
    assert rel_err(lp, rlp) <= RTOL
    assert rel_err(lse, rlse) <= RTOL


def test_logprob_shifted_view_and_unaligned_rows(pkg, gpu):
    c = _small_case(2, n_seq=2, n_tok=9, vocab=1003)
    lg = c["logits"].to(gpu)
    ids = c["ids"].to(gpu)
    print("[grpo] shifted view", flush=True)
    lp, _ = pkg.kernels.logprob_gather(lg[:, :-1], ids[:, 1:])
    torch.cuda.synchronize()
    rlp, _ = OG.logprob_gather(c["logits"][:, :-1], c["ids"][:, 1:])
    assert rel_err(lp, rlp) <= RTOL


def test_logprob_closed_forms_on_gpu(pkg, gpu):
    v = 151936
    logits = torch.full((1, 2, v), 0.5, dtype=torch.bfloat16, device=gpu)
    logits[0, 1, 77] = 80.0
    ids = torch.tensor([[3, 77]], device=gpu)
    print("[grpo] closed forms", flush=True)
    lp, lse = pkg.kernels.logprob_gather(logits, ids)
    torch.cuda.synchronize()
    assert abs(lp[0, 0].item() + math.log(v)) < 1e-4 * math.log(v)
    assert abs(lp[0, 1].item()) < 1e-5


def test_bad_token_id_gives_nan(pkg, gpu):
    logits = torch.zeros((1, 2, 64), dtype=torch.bfloat16, device=gpu)
    ids = torch.tensor([[-1, 64]], device=gpu)
    lp, _ = pkg.kernels.logprob_gather(logits, ids)
    torch.cuda.synchronize()
    assert torch.isnan(lp).all()


@pytest.mark.parametrize("eps", [1e-8, 1e-4])
def test_advantage_kernel(pkg, gpu, eps):
    r = torch.tensor([1., 0, 1, 0, 1, 0, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 0.3, 0.9, 0.1, 0.4])
    pid = torch.tensor([0] * 8 + [1] * 8 + [7, 2, 7, 2])
    print("[grpo] advantage", flush=True)
    a = pkg.kernels.grpo_advantage(r.to(gpu), pid.to(gpu), eps)
    torch.cuda.synchronize()
    ref = OG.advantage(r, pid, eps)
    assert rel_err(a, ref) <= RTOL


@pytest.mark.parametrize("reduction", ["token", "seq"])
@pytest.mark.parametrize("per_token_adv", [True, False])
def test_ppo_loss_kernel_and_grad(pkg, gpu, reduction, per_token_adv):
    c = _small_case(3)
    new, _ = OG.logprob_gather(c["logits"], c["ids"])
    adv = OG.advantage(c["rewards"], c["pids"])
    adv_tok = adv[:, None] * c["mask"]
    print(f"[grpo] ppo loss {reduction} per_token={per_token_adv}", flush=True)
    a_in = adv_tok if per_token_adv else adv
    loss, dlp = pkg.kernels.ppo_clipped_loss_fwd(new.to(gpu), c["old"].to(gpu), a_in.to(gpu),
                                                 c["mask"].to(gpu), 0.2, reduction)
    torch.cuda.synchronize()
    rloss, rgrad = OG.ppo_loss_and_grad(c["old"], new, adv_tok, c["mask"], 0.2, reduction)
    assert rel_err(loss, rloss) <= RTOL
    assert (dlp.cpu() - rgrad).abs().max().item() <= 1e-6 + 1e-4 * rgrad.abs().max().item()


@pytest.mark.parametrize("reduction", ["token", "seq"])
@pytest.mark.parametrize("adv_eps", [1e-8, 1e-4])
def test_fused_loss_matches_oracle(pkg, gpu, reduction, adv_eps):
    c = _small_case(4, n_seq=8, n_tok=33, vocab=1024)
    print(f"[grpo] fused {reduction} eps={adv_eps}", flush=True)
    res = pkg.kernels.grpo_fused_forward(c["logits"].to(gpu), c["ids"].to(gpu), c["old"].to(gpu),
                                         c["mask"].to(gpu), c["rewards"].to(gpu),
                                         c["pids"].to(gpu), adv_eps, 0.2, reduction)
    torch.cuda.synchronize()
    ref = OG.fused_loss_step(c["logits"], c["ids"], c["old"], c["mask"], c["rewards"], c["pids"],
                             adv_eps, 0.2, reduction)
    assert rel_err(res["lp"], ref["lp"]) <= RTOL
    assert rel_err(res["lse"], ref["lse"]) <= RTOL
    assert rel_err(res["adv"], ref["adv"]) <= RTOL
    assert rel_err(res["loss"], ref["loss"]) <= RTOL
    assert (res["dlp"].cpu() - ref["dlp"]).abs().max().item() <= 1e-4 * ref["dlp"].abs().max().item() + 1e-7
    # Second call reuses the cached workspace: the counters were reset.
    res2 = pkg.kernels.grpo_fused_forward(c["logits"].to(gpu), c["ids"].to(gpu), c["old"].to(gpu),
                                          c["mask"].to(gpu), c["rewards"].to(gpu),
                                          c["pids"].to(gpu), adv_eps, 0.2, reduction)
    torch.cuda.synchronize()
    assert torch.equal(res2["loss"], res["loss"]) and torch.equal(res2["dlp"], res["dlp"])


def test_backward_matches_autograd(pkg, gpu):
    c = _small_case(5, n_seq=4, n_tok=6, vocab=1000)
    g = torch.Generator().manual_seed(6)
    coef = torch.randn(4, 6, generator=g)
    coef[1, 2] = 0.0  # zero rows are written without reading logits
    lp, lse = OG.logprob_gather(c["logits"], c["ids"])
    print("[grpo] backward", flush=True)
    grad = pkg.kernels.logprob_gather_backward(c["logits"].to(gpu), c["ids"].to(gpu),
                                               lse.to(gpu), coef.to(gpu),
                                               torch.tensor(0.5, device=gpu))
    torch.cuda.synchronize()
    ref = OG.logits_grad(c["logits"], c["ids"], coef * 0.5)
    # bf16 output: compare within one bf16 ulp of the largest entry per row
    err = (grad.float().cpu() - ref).abs().max().item()
    assert err <= 2 ** -8 * ref.abs().max().item() + 1e-6
    assert grad[1, 2].abs().max().item() == 0.0


def test_grpo_config2_full_size(pkg, gpu):
    """Config 2 (32 x 512 rows, vocab 151936): all rows on the GPU against the
    oracle on a 96-row sample, plus the loss recomputed from the oracle's
    log-probabilities of every row."""
    print("[grpo] config2 generate", flush=True)
    w = W.grpo_loss_step(seed=0, device=gpu)
    print("[grpo] config2 fused", flush=True)
    res = pkg.kernels.grpo_fused_forward(w["logits"], w["ids"], w["old_lp"], w["mask"],
                                         w["rewards"], w["prompt_ids"], 1e-4, 0.2, "seq")
    torch.cuda.synchronize()
    # the generator's exact fp32 log-probabilities (torch.log_softmax on the GPU)
    assert rel_err(res["lp"], w["new_lp"]) <= RTOL
    g = torch.Generator().manual_seed(7)
    rows = torch.randperm(32 * 512, generator=g)[:96]
    sample = w["logits"].view(-1, 151936)[rows.to(gpu)].cpu()
    rlp, rlse = OG.logprob_gather(sample, w["ids"].view(-1)[rows.to(gpu)].cpu())
    assert rel_err(res["lp"].view(-1)[rows.to(gpu)], rlp) <= RTOL
    assert rel_err(res["lse"].view(-1)[rows.to(gpu)], rlse) <= RTOL
    adv = OG.advantage(w["rewards"].cpu(), w["prompt_ids"].cpu(), 1e-4)
    rloss, rgrad = OG.ppo_loss_and_grad(w["old_lp"].cpu(), w["new_lp"].cpu(),
                                        adv[:, None] * w["mask"].cpu(), w["mask"].cpu(), 0.2, "seq")
    assert rel_err(res["adv"], adv) <= RTOL
    assert rel_err(res["loss"], rloss) <= RTOL


@pytest.mark.parametrize("reduction", ["token", "seq"])
def test_loss_with_empty_and_single_token_responses(pkg, gpu, reduction):
    """A sequence whose response mask is all zero contributes 0 to either
    reduction (its mask sum gets the reference's + 1e-8, so no 0/0) and gets a
    zero gradient; a one-token response is an ordinary mean over one token.
    Fused (log-probs from logits) and plain forms against the oracle."""
    c = _small_case(9, n_seq=8, n_tok=12, vocab=1001)
    c["mask"][2] = 0.0                 # empty response
    c["mask"][5] = 0.0
    c["mask"][5, 0] = 1.0              # a single response token
    print(f"[grpo] empty / single-token responses ({reduction})", flush=True)
    res = pkg.kernels.grpo_fused_forward(c["logits"].to(gpu), c["ids"].to(gpu), c["old"].to(gpu),
                                         c["mask"].to(gpu), c["rewards"].to(gpu),
                                         c["pids"].to(gpu), 1e-4, 0.2, reduction)
    new, _ = OG.logprob_gather(c["logits"], c["ids"])
    adv = OG.advantage(c["rewards"], c["pids"], 1e-4)
    adv_tok = adv[:, None] * c["mask"]
    loss, dlp = pkg.kernels.ppo_clipped_loss_fwd(new.to(gpu), c["old"].to(gpu), adv_tok.to(gpu),
                                                 c["mask"].to(gpu), 0.2, reduction)
    torch.cuda.synchronize()
    ref = OG.fused_loss_step(c["logits"], c["ids"], c["old"], c["mask"], c["rewards"], c["pids"],
                             1e-4, 0.2, reduction)
    assert torch.isfinite(res["loss"]).all() and torch.isfinite(loss).all()
    assert rel_err(res["loss"], ref["loss"]) <= RTOL and rel_err(loss, ref["loss"]) <= RTOL
    tol = 1e-4 * ref["dlp"].abs().max().item() + 1e-7
    assert (res["dlp"].cpu() - ref["dlp"]).abs().max().item() <= tol
    assert (dlp.cpu() - ref["dlp"]).abs().max().item() <= tol
    assert (res["dlp"].cpu()[2] == 0).all() and (dlp.cpu()[2] == 0).all()
