"""GRPO loss step on the gfx950 kernels, with the call surface of
qwen3-naive-inference's qwen3_grpo_train.py:

  forward_logprob(model, input_ids)                  :46-53
  compute_grpo_advantage(rewards, prompt_ids)        :162-173
  ppo_clipped_loss(old, new, advantages, mask)       :184-199
  grpo_train_step(model, optimizer, input_ids, old_log_probs, response_mask,
                  rewards, prompt_ids)               :261-286

plus the fused paths.  ``grpo_loss_from_hidden`` (and ``forward_logprob``
without autograd) run the lm_head inside the log-softmax kernel, so no logits
exist at all.  ``grpo_fused_loss`` / ``grpo_fused_train_step``: one
streaming pass over the bf16 logits computes every token's log-probability,
the group advantages and the clipped masked loss, and its backward writes the
bf16 logit gradients directly, so the fp32 ``[B, T, V]`` log-softmax the
reference materialises (twice 9.96 GB at 32x512x151936) never exists.

Alignment: ``forward_logprob`` keeps the reference's unshifted gather
(position t's logits with token t).  The fused path takes ``shift=True`` for
next-token alignment (logits[:, t-1] with ids[:, t]).
"""
from __future__ import annotations

import torch

from . import kernels as K

CLIP_EPSILON = 0.2
PPO_EPOCHS = 1
ADV_EPS = 1e-8


class LogprobGather(torch.autograd.Function):
    """lp[b,t] = log_softmax(float(logits[b,t]))[ids[b,t]] with a HIP backward."""

    @staticmethod
    def forward(ctx, logits, ids):
        lp, lse = K.logprob_gather(logits, ids)
        ctx.save_for_backward(logits, ids, lse)
        return lp

    @staticmethod
    def backward(ctx, grad_lp):
        logits, ids, lse = ctx.saved_tensors
        grad = K.logprob_gather_backward(logits, ids, lse, grad_lp.float().contiguous())
        return grad, None


class GrpoFusedLoss(torch.autograd.Function):
    """Loss of the whole GRPO step from bf16 logits (forward: one streaming pass;
    backward: d loss / d logits = g * dlp * (onehot - softmax))."""

    @staticmethod
    def forward(ctx, logits, ids, old_lp, mask, rewards, prompt_ids, adv_eps, clip, reduction):
        res = K.grpo_fused_forward(logits, ids, old_lp, mask, rewards, prompt_ids, adv_eps, clip,
                                   reduction)
        ctx.save_for_backward(logits, ids, res["lse"], res["dlp"])
        ctx.mark_non_differentiable(res["lp"], res["adv"])
        return res["loss"], res["lp"], res["adv"]

    @staticmethod
    def backward(ctx, grad_loss, _glp, _gadv):
        logits, ids, lse, dlp = ctx.saved_tensors
        g = grad_loss.reshape(1).float().contiguous()
        grad = K.logprob_gather_backward(logits, ids, lse, dlp, grad_scale=g)
        return grad, None, None, None, None, None, None, None, None


class PpoClippedLoss(torch.autograd.Function):
    """Clipped surrogate on given log-probabilities with a HIP forward/backward."""

    @staticmethod
    def forward(ctx, new_lp, old_lp, adv, mask, clip, reduction):
        loss, dlp = K.ppo_clipped_loss_fwd(new_lp, old_lp, adv, mask, clip, reduction,
                                           need_grad=True)
        ctx.save_for_backward(dlp)
        ctx.shape = new_lp.shape
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        (dlp,) = ctx.saved_tensors
        return (dlp * grad_loss).reshape(ctx.shape), None, None, None, None, None


# ---------------------------------------------------------------------------
def forward_logprob(model, input_ids):
    """Per-position log-probability of ``input_ids`` under ``model`` (unshifted,
    as the reference gathers position t's logits at token t).

    Without autograd the lm_head and the gather run fused (``lm_head_logprob``:
    the logits rounded to bf16 as the lm_head's output is, never
    materialised); with autograd the bf16 logits are materialised and the
    gather has a HIP backward."""
    weight = getattr(getattr(model, "lm_head", None), "weight", None)
    if (not torch.is_grad_enabled() and weight is not None and weight.is_cuda
            and weight.dtype == torch.bfloat16 and hasattr(model, "model")):
        hidden = model.model(input_ids)
        lp, _ = K.lm_head_logprob(hidden.reshape(-1, hidden.shape[-1]), weight,
                                  input_ids.reshape(-1))
        return lp.view(input_ids.shape)
    logits = model(input_ids)
    return LogprobGather.apply(logits, input_ids)


def grpo_loss_from_hidden(hidden, lm_head_weight, ids, old_log_probs, response_mask, rewards,
                          prompt_ids, adv_eps: float = ADV_EPS,
                          clip_epsilon: float = CLIP_EPSILON, reduction: str = "token",
                          shift: bool = False):
    """Forward-only GRPO loss step from final hidden states ``[B, T, H]``: each
    token's log-probability by the fused lm_head kernel (the ``[B, T, V]``
    logits never exist), group advantages and the clipped masked loss.
    Returns (loss, lp ``[B, T']``, adv ``[B]``); ``shift`` as in grpo_fused_loss."""
    if shift:
        hidden, ids = hidden[:, :-1], ids[:, 1:]
        old_log_probs = old_log_probs[:, 1:]
        response_mask = response_mask[:, 1:]
    bsz, t = ids.shape
    lp, _ = K.lm_head_logprob(hidden.reshape(bsz * t, -1), lm_head_weight, ids.reshape(-1))
    lp = lp.view(bsz, t)
    adv = K.grpo_advantage(rewards, prompt_ids, adv_eps)
    loss, _ = K.ppo_clipped_loss_fwd(lp, old_log_probs.float(), adv, response_mask.float(),
                                     clip_epsilon, reduction, need_grad=False)
    return loss, lp, adv


def compute_grpo_advantage(rewards, prompt_ids, eps: float = ADV_EPS):
    """(r - mean_g) / (std_g + eps) within each prompt group (unbiased std)."""
    out = K.grpo_advantage(rewards, prompt_ids, eps)
    return out.to(rewards.dtype) if rewards.is_floating_point() else out


def ppo_clipped_loss(old_log_probs, new_log_probs, advantages, response_mask,
                     clip_epsilon: float = CLIP_EPSILON, reduction: str = "token"):
    """-min(r A, clamp(r, 1-e, 1+e) A), token-masked mean (``reduction="seq"``:
    mean over sequences of each sequence's masked mean)."""
    return PpoClippedLoss.apply(new_log_probs, old_log_probs, advantages, response_mask,
                                clip_epsilon, reduction)


def grpo_train_step(model, optimizer, input_ids, old_log_probs, response_mask, rewards,
                    prompt_ids, ppo_epochs: int = PPO_EPOCHS, clip_epsilon: float = CLIP_EPSILON):
    """Advantages -> PPO epochs of {forward_logprob, clipped loss, backward, step}."""
    advantages = compute_grpo_advantage(rewards.float(), prompt_ids)
    token_advantages = advantages[:, None] * response_mask.float()
    total = torch.zeros((), device=input_ids.device)
    for _ in range(ppo_epochs):
        new_log_probs = forward_logprob(model, input_ids)
        loss = ppo_clipped_loss(old_log_probs, new_log_probs, token_advantages, response_mask,
                                clip_epsilon)
        optimizer.zero_grad()
        loss.backward()
        optimizer.step()
        total += loss.detach()
    return (total / ppo_epochs).item()


def grpo_fused_loss(logits, ids, old_log_probs, response_mask, rewards, prompt_ids,
                    adv_eps: float = ADV_EPS, clip_epsilon: float = CLIP_EPSILON,
                    reduction: str = "token", shift: bool = False):
    """Fused loss step from ``[B, T, V]`` bf16 logits.  Returns (loss, lp, adv).

    ``shift=True`` pairs logits[:, t-1] with ids[:, t] (next-token alignment);
    old_log_probs / response_mask then refer to positions 1..T-1.
    """
    if shift:
        logits, ids = logits[:, :-1], ids[:, 1:]
        old_log_probs = old_log_probs[:, 1:]
        response_mask = response_mask[:, 1:]
    return GrpoFusedLoss.apply(logits, ids, old_log_probs, response_mask, rewards, prompt_ids,
                               adv_eps, clip_epsilon, reduction)


def grpo_fused_train_step(model, optimizer, input_ids, old_log_probs, response_mask, rewards,
                          prompt_ids, ppo_epochs: int = PPO_EPOCHS,
                          clip_epsilon: float = CLIP_EPSILON, adv_eps: float = ADV_EPS,
                          reduction: str = "token", shift: bool = False):
    """grpo_train_step with the fused kernel between the model and the loss."""
    total = torch.zeros((), device=input_ids.device)
    for _ in range(ppo_epochs):
        logits = model(input_ids)
        loss, _, _ = grpo_fused_loss(logits, input_ids, old_log_probs, response_mask, rewards,
                                     prompt_ids, adv_eps, clip_epsilon, reduction, shift)
        optimizer.zero_grad()
        loss.backward()
        optimizer.step()
        total += loss.detach()
    return (total / ppo_epochs).item()
