"""Pins the oracle's GRPO loss step (CPU): closed forms, library routines,
finite differences and hand-computed cases."""
import math

import pytest
import torch

from oracle import grpo


def test_logprob_equal_logits_is_minus_log_v():
    v = 151936
    logits = torch.full((2, 3, v), 0.75, dtype=torch.bfloat16)
    ids = torch.tensor([[0, 5, v - 1], [7, 8, 9]])
    lp, lse = grpo.logprob_gather(logits, ids)
    torch.testing.assert_close(lp, torch.full((2, 3), -math.log(v)), atol=1e-5, rtol=0)
    torch.testing.assert_close(lse, torch.full((2, 3), 0.75 + math.log(v)), atol=1e-5, rtol=0)


def test_logprob_one_hot_and_normalisation():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(4, 1000, generator=g).to(torch.bfloat16)
    logits[0, 17] = 60.0
    ids = torch.tensor([17, 3, 999, 0])
    lp, lse = grpo.logprob_gather(logits, ids)
    assert abs(lp[0].item()) < 1e-6
    # sum_v exp(lp_v) == 1 on every row (through the lse it returns)
    full = logits.float() - lse[:, None]
    torch.testing.assert_close(full.exp().sum(-1), torch.ones(4), atol=1e-5, rtol=0)
    # and it equals torch.log_softmax (library routine) gathered.
    ref = torch.log_softmax(logits.double(), -1).gather(-1, ids[:, None])[:, 0]
    torch.testing.assert_close(lp.double(), ref, atol=1e-5, rtol=0)


def test_advantage_closed_form():
    # Four 1s and four 0s: mean 0.5, unbiased std sqrt(2/7) -> +-0.5/sqrt(2/7).
    r = torch.tensor([1., 0, 1, 0, 1, 0, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1])
    pid = torch.tensor([0] * 8 + [1] * 8)
    a = grpo.advantage(r, pid, eps=1e-8)
    expect = 0.5 / (math.sqrt(2 / 7) + 1e-8)
    torch.testing.assert_close(a[:8], torch.tensor([expect, -expect] * 4), atol=1e-6, rtol=0)
    # All-equal group -> 0 (std 0, numerator 0).
    torch.testing.assert_close(a[8:], torch.zeros(8))
    a4 = grpo.advantage(r, pid, eps=1e-4)
    assert abs(a4[0].item() - 0.5 / (math.sqrt(2 / 7) + 1e-4)) < 1e-6


def test_advantage_noncontiguous_groups_and_singleton():
    r = torch.tensor([1., 5, 3, 7])
    pid = torch.tensor([4, 9, 4, 2])
    a = grpo.advantage(r, pid)
    m, s = 2.0, math.sqrt(2.0)
    torch.testing.assert_close(a[[0, 2]], torch.tensor([(1 - m) / (s + 1e-8), (3 - m) / (s + 1e-8)]))
    assert math.isnan(a[1].item()) and math.isnan(a[3].item())  # torch.std of one value


def _loss_by_hand(old, new, adv, mask, clip, reduction):
    per = []
    for b in range(len(old)):
        row = []
        for t in range(len(old[b])):
            r = math.exp(new[b][t] - old[b][t])
            rc = min(max(r, 1 - clip), 1 + clip)
            row.append(-min(r * adv[b][t], rc * adv[b][t]) * mask[b][t])
        per.append(row)
    if reduction == "token":
        return sum(map(sum, per)) / (sum(map(sum, mask)) + 1e-8)
    return sum(sum(per[b]) / (sum(mask[b]) + 1e-8) for b in range(len(per))) / len(per)


@pytest.mark.parametrize("reduction", ["token", "seq"])
def test_loss_hand_cases(reduction):
    # Inside the clip range, clipped above (A>0), clipped below (A<0), masked.
    old = [[0.0, 0.0, 0.0], [-1.0, -2.0, 0.0]]
    new = [[0.1, 0.5, -0.5], [-1.05, -1.0, 3.0]]
    adv = [[1.0, 1.0, 1.0], [-2.0, -2.0, -2.0]]
    mask = [[1.0, 1.0, 1.0], [1.0, 1.0, 0.0]]
    t = lambda x: torch.tensor(x, dtype=torch.float32)
    loss = grpo.ppo_loss(t(old), t(new), t(adv), t(mask), 0.2, reduction)
    assert abs(loss.item() - _loss_by_hand(old, new, adv, mask, 0.2, reduction)) < 1e-6


@pytest.mark.parametrize("reduction", ["token", "seq"])
def test_loss_gradient_matches_finite_differences(reduction):
    g = torch.Generator().manual_seed(1)
    old = torch.randn(3, 7, generator=g, dtype=torch.float64) * 0.3
    new = old + torch.randn(3, 7, generator=g, dtype=torch.float64) * 0.4
    adv = torch.randn(3, 1, generator=g, dtype=torch.float64).expand(3, 7).clone()
    mask = (torch.rand(3, 7, generator=g) > 0.3).double()
    nw = new.clone().requires_grad_(True)
    grpo.ppo_loss(old, nw, adv, mask, 0.2, reduction).backward()
    h = 1e-6
    for b in range(3):
        for t in range(7):
            e = torch.zeros_like(new)
            e[b, t] = h
            fd = (grpo.ppo_loss(old, new + e, adv, mask, 0.2, reduction)
                  - grpo.ppo_loss(old, new - e, adv, mask, 0.2, reduction)) / (2 * h)
            r = math.exp(new[b, t] - old[b, t])
            if abs(r - 0.8) > 1e-4 and abs(r - 1.2) > 1e-4:  # away from the kinks
                assert abs(fd.item() - nw.grad[b, t].item()) < 1e-6


def test_loss_gradient_closed_form():
    # d/dnew of -min(rA, clip(r)A) = -A r where the unclipped branch is active.
    old = torch.zeros(1, 4)
    new = torch.tensor([[0.0, 0.5, -0.5, 0.1]])  # r = 1, 1.65 (clip), 0.61 (clip), 1.105
    adv = torch.tensor([[1.0, 1.0, 1.0, -1.0]])
    mask = torch.ones(1, 4)
    loss, grad = grpo.ppo_loss_and_grad(old, new, adv, mask, 0.2, "token")
    r = new.exp()
    # A>0: r=1.65>1.2 -> clipped (min picks clipped) -> 0;  r=0.61<0.8 -> min picks r*A -> -A r
    expect = torch.tensor([[-1.0, 0.0, -r[0, 2].item(), r[0, 3].item()]]) / 4
    torch.testing.assert_close(grad, expect, atol=1e-6, rtol=0)


def test_logits_grad_formula():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 3, 50, generator=g)
    ids = torch.randint(0, 50, (2, 3), generator=g)
    coef = torch.randn(2, 3, generator=g)
    grad = grpo.logits_grad(x, ids, coef)
    p = torch.softmax(x, -1)
    onehot = torch.nn.functional.one_hot(ids, 50).float()
    torch.testing.assert_close(grad, coef[..., None] * (onehot - p), atol=1e-6, rtol=0)
