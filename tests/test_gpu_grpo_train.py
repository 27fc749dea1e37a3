"""GRPO training step on the GPU: the reference surface (forward_logprob +
ppo_clipped_loss + backward) and the fused path give the same loss and the
same parameter gradients as torch autograd through the reference's formulas
(log_softmax(logits.float()).gather, PPO clip, token-masked mean)."""
import pytest
import torch

from oracle import grpo as OG

pytestmark = pytest.mark.gpu


def _setup(pkg, gpu):
    # Untied lm_head: with tied embeddings a random model puts p ~ 1 on the
    # input token itself, and the unshifted gather (position t scored at token
    # t, as the reference does) would then have a vanishing gradient.
    cfg = pkg.Qwen3Config(num_hidden_layers=2, vocab_size=1024, tie_word_embeddings=False)
    torch.manual_seed(0)
    m = pkg.Qwen3ForCausalLM(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.uniform_(0.8, 1.2)
            elif "embed" in name:
                p.normal_(0, 0.25)
            elif "lm_head" in name:
                p.normal_(0, 0.05)
            elif p.dim() == 2:
                p.normal_(0, 0.02)
    m = m.to(gpu).to(torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    b, t = 4, 48
    ids = torch.randint(0, 1024, (b, t), generator=g).to(gpu)
    lens = torch.tensor([20, 48, 33, 9])
    mask = ((torch.arange(t)[None] >= 8) & (torch.arange(t)[None] < 8 + lens[:, None])).float().to(gpu)
    with torch.no_grad():
        lp0 = torch.log_softmax(m(ids).float(), -1).gather(-1, ids[..., None])[..., 0]
    old = (lp0 + 0.1 * torch.randn(b, t, generator=g).to(gpu)) * mask
    rewards = torch.tensor([1.0, 0.0, 0.0, 1.0], device=gpu)
    pids = torch.tensor([0, 0, 1, 1], device=gpu)
    return m, ids, old, mask, rewards, pids


def _grads(m):
    g = torch.cat([p.grad.float().reshape(-1) for p in m.parameters() if p.grad is not None])
    assert g.norm() > 1e-3, "degenerate setup: vanishing gradient"
    return g


def _reference_step(m, ids, old, mask, rewards, pids):
    """torch autograd through the reference's own formulas (fp32 loss math)."""
    m.zero_grad()
    logits = m(ids)
    lp = torch.log_softmax(logits.float(), dim=-1).gather(-1, ids[..., None])[..., 0]
    adv = OG.advantage(rewards.cpu(), pids.cpu()).to(ids.device)
    loss = OG.ppo_loss(old, lp, adv[:, None] * mask, mask, 0.2, "token")
    loss.backward()
    return loss.detach(), _grads(m)


def test_reference_surface_matches_autograd(pkg, gpu):
    m, ids, old, mask, rewards, pids = _setup(pkg, gpu)
    print("[grpo-train] reference surface", flush=True)
    rloss, rgrad = _reference_step(m, ids, old, mask, rewards, pids)
    m.zero_grad()
    adv = pkg.compute_grpo_advantage(rewards, pids)
    new = pkg.forward_logprob(m, ids)
    loss = pkg.ppo_clipped_loss(old, new, adv[:, None] * mask, mask)
    loss.backward()
    grad = _grads(m)
    assert abs(loss.item() - rloss.item()) <= 1e-4 * max(1.0, abs(rloss.item()))
    cos = torch.nn.functional.cosine_similarity(grad, rgrad, dim=0).item()
    assert cos > 0.9999 and (grad - rgrad).norm() / rgrad.norm() < 1e-2


@pytest.mark.parametrize("reduction", ["token", "seq"])
def test_fused_loss_matches_autograd(pkg, gpu, reduction):
    m, ids, old, mask, rewards, pids = _setup(pkg, gpu)
    print(f"[grpo-train] fused {reduction}", flush=True)
    m.zero_grad()
    logits = m(ids)
    lp = torch.log_softmax(logits.float(), -1).gather(-1, ids[..., None])[..., 0]
    adv = OG.advantage(rewards.cpu(), pids.cpu()).to(gpu)
    rloss = OG.ppo_loss(old, lp, adv[:, None] * mask, mask, 0.2, reduction)
    rloss.backward()
    rgrad = _grads(m)
    m.zero_grad()
    loss, lp2, adv2 = pkg.grpo_fused_loss(m(ids), ids, old, mask, rewards, pids, 1e-8, 0.2,
                                          reduction)
    loss.backward()
    grad = _grads(m)
    assert abs(loss.item() - rloss.item()) <= 1e-4 * max(1.0, abs(rloss.item()))
    assert ((lp2 - lp.detach()).abs() / lp.detach().abs().clamp_min(1)).max().item() <= 1e-4
    cos = torch.nn.functional.cosine_similarity(grad, rgrad, dim=0).item()
    assert cos > 0.9999 and (grad - rgrad).norm() / rgrad.norm() < 1e-2


def test_train_steps_update_parameters(pkg, gpu):
    m, ids, old, mask, rewards, pids = _setup(pkg, gpu)
    opt = torch.optim.AdamW(m.parameters(), lr=1e-3)
    before = m.model.layers[0].mlp.down_proj.weight.detach().clone()
    print("[grpo-train] train steps", flush=True)
    l1 = pkg.grpo_train_step(m, opt, ids, old, mask, rewards, pids)
    l2 = pkg.grpo_fused_train_step(m, opt, ids, old, mask, rewards, pids)
    assert all(map(lambda v: v == v and abs(v) < 1e3, (l1, l2)))
    assert not torch.equal(before, m.model.layers[0].mlp.down_proj.weight)
