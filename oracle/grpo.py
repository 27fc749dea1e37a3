"""GRPO loss step restated on the CPU in fp32.

Reference: qwen3_grpo_train.py
  forward_logprob          :46-53   log_softmax(logits.float()).gather(ids), unshifted
  compute_grpo_advantage   :162-173 per unique prompt id: (r - mean) / (std + 1e-8),
                                    std unbiased (torch default)
  token advantages         :269     A[:, None] * response_mask
  ppo_clipped_loss         :184-199 ratio = exp(new - old); -min(ratio*A, clamp(ratio)*A);
                                    sum(l * m) / (sum(m) + 1e-8)
The loss is written with torch ops on fp32 CPU tensors so autograd gives the
gradient the reference's loss.backward() (:281) would compute.
Extra reduction "seq": mean over sequences of sum_t(l*m) / (sum_t(m) + 1e-8),
the per-sequence masked mean of the GRPO loss-step workload.
"""
from __future__ import annotations

import torch


def logprob_gather(logits: torch.Tensor, ids: torch.Tensor, chunk_rows: int = 512):
    """fp32 ``(lp, lse)`` of ``log_softmax(float(logits)).gather(ids)``.

    ``logits [..., V]`` and ``ids [...]``; processed in row chunks to bound RAM.
    """
    v = logits.shape[-1]
    flat = logits.reshape(-1, v)
    fid = ids.reshape(-1)
    lp = torch.empty(fid.shape[0], dtype=torch.float32)
    lse = torch.empty(fid.shape[0], dtype=torch.float32)
    for s in range(0, flat.shape[0], chunk_rows):
        x = flat[s:s + chunk_rows].float()
        l = torch.logsumexp(x, dim=-1)
        lse[s:s + chunk_rows] = l
        lp[s:s + chunk_rows] = x.gather(-1, fid[s:s + chunk_rows, None])[:, 0] - l
    return lp.view(ids.shape), lse.view(ids.shape)


def advantage(rewards: torch.Tensor, prompt_ids: torch.Tensor, eps: float = 1e-8) -> torch.Tensor:
    """Group-normalised advantages, one Python pass per unique prompt id."""
    r = rewards.float()
    out = torch.empty_like(r)
    for pid in prompt_ids.unique():
        m = prompt_ids == pid
        g = r[m]
        out[m] = (g - g.mean()) / (g.std() + eps)
    return out


def ppo_loss(old_lp: torch.Tensor, new_lp: torch.Tensor, adv_tok: torch.Tensor,
             mask: torch.Tensor, clip: float = 0.2, reduction: str = "token") -> torch.Tensor:
    """Clipped surrogate; differentiable w.r.t. ``new_lp``."""
    ratio = (new_lp - old_lp).exp()
    clipped = ratio.clamp(1.0 - clip, 1.0 + clip)
    per_tok = -torch.min(ratio * adv_tok, clipped * adv_tok)
    if reduction == "token":
        return (per_tok * mask).sum() / (mask.sum() + 1e-8)
    if reduction == "seq":
        return ((per_tok * mask).sum(-1) / (mask.sum(-1) + 1e-8)).mean()
    raise ValueError(reduction)


def ppo_loss_and_grad(old_lp, new_lp, adv_tok, mask, clip=0.2, reduction="token"):
    """Loss and d loss / d new_lp via autograd (fp32, CPU)."""
    nw = new_lp.detach().float().clone().requires_grad_(True)
    loss = ppo_loss(old_lp.float(), nw, adv_tok.float(), mask.float(), clip, reduction)
    loss.backward()
    return loss.detach(), nw.grad.detach()


def fused_loss_step(logits, ids, old_lp, mask, rewards, prompt_ids, adv_eps=1e-8, clip=0.2,
                    reduction="token"):
    """Reference composition of the fused kernel's outputs (fp32)."""
    lp, lse = logprob_gather(logits, ids)
    adv = advantage(rewards, prompt_ids, adv_eps)
    adv_tok = adv[:, None] * mask.float()
    loss, dlp = ppo_loss_and_grad(old_lp, lp, adv_tok, mask, clip, reduction)
    return {"loss": loss, "lp": lp, "lse": lse, "dlp": dlp, "adv": adv}


def logits_grad(logits: torch.Tensor, ids: torch.Tensor, coef: torch.Tensor) -> torch.Tensor:
    """d/d logits of sum(coef * lp) through log_softmax(logits.float()) (fp32)."""
    x = logits.detach().float().requires_grad_(True)
    lp = torch.log_softmax(x, dim=-1).gather(-1, ids[..., None])[..., 0]
    (lp * coef.float()).sum().backward()
    return x.grad.detach()
