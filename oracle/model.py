"""Qwen3 forward restated on the CPU in fp32 (or float64) from a state dict.

Reference: qwen3_naive.py, the eager no-cache batch forward
  Qwen3ForCausalLM.forward -> Qwen3Model.forward -> Qwen3DecoderLayer.forward
  -> Qwen3Attention.forward (batch path, :553-593), RMSNorm (:156-161),
  RoPE (:44-67, :380-387), Qwen3MLP (:695-702), tied lm_head (:826-835).
Weights are inputs (the state dict of a model under test), so the oracle
needs no checkpoint.  Parameter names follow the reference module tree.
"""
from __future__ import annotations

import torch

from . import norm_rope as NR


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def qwen3_logits(sd: dict, input_ids: torch.Tensor, n_layers: int, n_heads: int = 16,
                 n_kv: int = 8, head_dim: int = 128, eps: float = 1e-6, theta: float = 1e6,
                 dtype=torch.float32) -> torch.Tensor:
    """Logits [B, T, V] of ``input_ids`` [B, T] (causal, positions 0..T-1)."""
    p = {k: v.detach().to("cpu", dtype) for k, v in sd.items()}
    bsz, t = input_ids.shape
    x = p["model.embed_tokens.weight"][input_ids]
    cache = NR.rope_cache(head_dim, max(t, 1), theta).to(dtype)
    pos = torch.arange(t)
    rep = n_heads // n_kv
    qs, ks = n_heads * head_dim, n_kv * head_dim
    mask = torch.triu(torch.ones(t, t, dtype=torch.bool), 1)
    for i in range(n_layers):
        pre = f"model.layers.{i}."
        h = _rms(x, p[pre + "input_layernorm.weight"], eps)
        qkv = h @ p[pre + "self_attn.qkv_proj.weight"].T
        q, k, v = qkv.split([qs, ks, ks], dim=-1)
        q = _rms(q.view(bsz, t, n_heads, head_dim), p[pre + "self_attn.q_norm.weight"], eps)
        k = _rms(k.view(bsz, t, n_kv, head_dim), p[pre + "self_attn.k_norm.weight"], eps)
        v = v.view(bsz, t, n_kv, head_dim)
        q = torch.stack([NR.apply_rope(q[b], pos, cache, dtype) for b in range(bsz)])
        k = torch.stack([NR.apply_rope(k[b], pos, cache, dtype) for b in range(bsz)])
        qh = q.transpose(1, 2)
        kh = k.transpose(1, 2).repeat_interleave(rep, 1)
        vh = v.transpose(1, 2).repeat_interleave(rep, 1)
        s = (qh @ kh.transpose(-2, -1)) * head_dim ** -0.5
        s = s.masked_fill(mask, float("-inf"))
        o = (torch.softmax(s, -1) @ vh).transpose(1, 2).reshape(bsz, t, qs)
        x = x + o @ p[pre + "self_attn.o_proj.weight"].T
        h = _rms(x, p[pre + "post_attention_layernorm.weight"], eps)
        gu = h @ p[pre + "mlp.gate_up_proj.weight"].T
        g, u = gu.chunk(2, dim=-1)
        x = x + (torch.nn.functional.silu(g) * u) @ p[pre + "mlp.down_proj.weight"].T
    x = _rms(x, p["model.norm.weight"], eps)
    head = p.get("lm_head.weight", p["model.embed_tokens.weight"])
    return x @ head.T
