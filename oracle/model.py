"""Qwen3 forward restated on the CPU from a state dict (test infrastructure).

Reference: qwen3_naive.py
  Qwen3ForCausalLM.forward -> Qwen3Model.forward -> Qwen3DecoderLayer.forward
  -> Qwen3Attention.forward (batch path, :553-593), RMSNorm (:156-169),
  RoPE (:44-67, :380-387), Qwen3MLP (:695-702), tied lm_head (:826-835);
  the paged decode step Qwen3Model.forward_decode (:795-802) with
  Qwen3DecoderLayer.forward_decode (:747-756) and
  Qwen3Attention.forward_decode (:642-683).
Weights are inputs (the state dict of a model under test), so the oracle
needs no checkpoint.  Parameter names follow the reference module tree.

Two arithmetic modes:
  "fp32"  exact math in ``dtype`` (fp32 or float64): no rounding anywhere.
  "bf16"  the reference's own bf16 model numerics, with every tensor the
          reference materialises in bf16 rounded there: the projection GEMM
          outputs (fp32 accumulation), RMSNorm and add+RMSNorm outputs and the
          bf16 residual they return (:156-169: fp32 math, one cast back; the
          norm of an add is taken of the fp32 sum), the QK-norm output and
          the RoPE output (:57-67, fp32 rotation of the bf16 normed values),
          the attention output, SwiGLU's silu(gate) * up (one rounding: the
          reference compiles the MLP with inductor, :695-702) and the logits.
          Attention itself is fp32 softmax(q k^T / sqrt(d)) v of the bf16
          q/k/v (flash-attn's semantics).
In fp32 mode the residual stream is carried unrounded, which makes the
layer loop the textbook pre-norm transformer; the bf16 mode only inserts
roundings into the same loop.
"""
from __future__ import annotations

import torch

from . import norm_rope as NR


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _params(sd, dtype):
    return {k: v.detach().to("cpu", dtype) for k, v in sd.items()}


def _rounder(mode: str, dtype):
    if mode == "fp32":
        return lambda t: t
    if mode == "bf16":
        return lambda t: t.to(torch.bfloat16).to(dtype)
    raise ValueError(mode)


def _qkv(p, pre, h, pos, cache, n_heads, n_kv, head_dim, eps, R, dtype):
    """Projection, per-head QK-RMSNorm and RoPE of h [N, H] at positions [N]."""
    n = h.shape[0]
    qs, ks = n_heads * head_dim, n_kv * head_dim
    qkv = R(h @ p[pre + "self_attn.qkv_proj.weight"].T)
    q, k, v = qkv.split([qs, ks, ks], dim=-1)
    q = R(_rms(q.reshape(n, n_heads, head_dim), p[pre + "self_attn.q_norm.weight"], eps))
    k = R(_rms(k.reshape(n, n_kv, head_dim), p[pre + "self_attn.k_norm.weight"], eps))
    q = R(NR.apply_rope(q, pos, cache, dtype))
    k = R(NR.apply_rope(k, pos, cache, dtype))
    return q, k, v.reshape(n, n_kv, head_dim)


def _attn_out_mlp(p, pre, attn, r, eps, R):
    """o_proj, add + post-attention RMSNorm, SwiGLU MLP.  ``r`` is the residual
    stream entering the layer; returns (the MLP output, the residual after the
    attention add)."""
    o = R(attn @ p[pre + "self_attn.o_proj.weight"].T)
    s = o + r
    r = R(s)
    h = R(_rms(s, p[pre + "post_attention_layernorm.weight"], eps))
    gu = R(h @ p[pre + "mlp.gate_up_proj.weight"].T)
    g, u = gu.chunk(2, dim=-1)
    a = R(torch.nn.functional.silu(g) * u)
    return R(a @ p[pre + "mlp.down_proj.weight"].T), r


def qwen3_forward_kv(sd: dict, input_ids: torch.Tensor, n_layers: int, n_heads: int = 16,
                     n_kv: int = 8, head_dim: int = 128, eps: float = 1e-6, theta: float = 1e6,
                     dtype=torch.float32, mode: str = "fp32"):
    """Causal forward of ``input_ids`` [B, T] (positions 0..T-1).

    Returns (logits [B, T, V], ks, vs) where ks[l] / vs[l] are layer l's keys
    (after QK-norm and RoPE) and values [B, T, n_kv, head_dim]: what the paged
    cache holds for these positions."""
    p = _params(sd, dtype)
    R = _rounder(mode, dtype)
    bsz, t = input_ids.shape
    cache = NR.rope_cache(head_dim, max(t, 1), theta).to(dtype)
    pos = torch.arange(t).repeat(bsz)
    rep = n_heads // n_kv
    mask = torch.triu(torch.ones(t, t, dtype=torch.bool), 1)
    r = R(p["model.embed_tokens.weight"][input_ids.reshape(-1)])      # [B*T, H]
    s = r
    ks, vs = [], []
    for i in range(n_layers):
        pre = f"model.layers.{i}."
        h = R(_rms(s, p[pre + "input_layernorm.weight"], eps))
        q, k, v = _qkv(p, pre, h, pos, cache, n_heads, n_kv, head_dim, eps, R, dtype)
        ks.append(k.view(bsz, t, n_kv, head_dim))
        vs.append(v.view(bsz, t, n_kv, head_dim))
        qh = q.view(bsz, t, n_heads, head_dim).transpose(1, 2)
        kh = k.view(bsz, t, n_kv, head_dim).transpose(1, 2).repeat_interleave(rep, 1)
        vh = v.view(bsz, t, n_kv, head_dim).transpose(1, 2).repeat_interleave(rep, 1)
        sc = (qh @ kh.transpose(-2, -1)) * head_dim ** -0.5
        sc = sc.masked_fill(mask, float("-inf"))
        attn = R((torch.softmax(sc, -1) @ vh).transpose(1, 2).reshape(bsz * t, n_heads * head_dim))
        d, r = _attn_out_mlp(p, pre, attn, r, eps, R)
        s = d + r
        r = R(s)
    x = R(_rms(s, p["model.norm.weight"], eps))
    head = p.get("lm_head.weight", p["model.embed_tokens.weight"])
    return R(x @ head.T).view(bsz, t, -1), ks, vs


def qwen3_logits(sd: dict, input_ids: torch.Tensor, n_layers: int, n_heads: int = 16,
                 n_kv: int = 8, head_dim: int = 128, eps: float = 1e-6, theta: float = 1e6,
                 dtype=torch.float32, mode: str = "fp32") -> torch.Tensor:
    """Logits [B, T, V] of ``input_ids`` [B, T] (causal, positions 0..T-1)."""
    return qwen3_forward_kv(sd, input_ids, n_layers, n_heads, n_kv, head_dim, eps, theta,
                            dtype, mode)[0]


def qwen3_decode_layer(sd: dict, layer: int, d_in, r_in, positions, k_ctx, v_ctx,
                       n_heads: int = 16, n_kv: int = 8, head_dim: int = 128, eps: float = 1e-6,
                       theta: float = 1e6, dtype=torch.float32, mode: str = "fp32", p=None):
    """One decoder layer of the decode step (Qwen3DecoderLayer.forward_decode,
    qwen3_naive.py:747-756): input (d_in, r_in) as the layer receives it --
    the previous layer's MLP output and the residual stream (d_in None for
    layer 0, whose input is the embedding r_in).  ``k_ctx[b]`` / ``v_ctx[b]``:
    the layer's cached rows [ctx_b, n_kv, D].  Returns (MLP output, residual,
    new_k [B, n_kv, D], new_v [B, n_kv, D])."""
    p = _params(sd, dtype) if p is None else p
    R = _rounder(mode, dtype)
    pos = torch.as_tensor(positions).long().view(-1)
    cache = NR.rope_cache(head_dim, int(pos.max()) + 1, theta).to(dtype)
    rep = n_heads // n_kv
    r = R(r_in.to(dtype))
    s = r if d_in is None else d_in.to(dtype) + r
    r = R(s)
    pre = f"model.layers.{layer}."
    h = R(_rms(s, p[pre + "input_layernorm.weight"], eps))
    q, k, v = _qkv(p, pre, h, pos, cache, n_heads, n_kv, head_dim, eps, R, dtype)
    outs = []
    for b in range(q.shape[0]):
        kk = torch.cat([k_ctx[b].to(dtype), k[b:b + 1]], 0)             # [ctx+1, n_kv, D]
        vv = torch.cat([v_ctx[b].to(dtype), v[b:b + 1]], 0)
        kh = kk.permute(1, 0, 2).repeat_interleave(rep, 0)               # [Hq, ctx+1, D]
        vh = vv.permute(1, 0, 2).repeat_interleave(rep, 0)
        sc = (kh @ q[b][:, :, None])[..., 0] * head_dim ** -0.5          # [Hq, ctx+1]
        outs.append((torch.softmax(sc, -1)[:, None, :] @ vh)[:, 0, :].reshape(-1))
    attn = R(torch.stack(outs))
    d, r = _attn_out_mlp(p, pre, attn, r, eps, R)
    return d, r, k, v


def qwen3_decode_step(sd: dict, token_ids, positions, k_ctx, v_ctx, n_layers: int,
                      n_heads: int = 16, n_kv: int = 8, head_dim: int = 128, eps: float = 1e-6,
                      theta: float = 1e6, dtype=torch.float32, mode: str = "fp32"):
    """One decode step per sequence (Qwen3Model.forward_decode, :795-802): the
    new token of sequence b at ``positions[b]`` attends to its cached keys
    plus itself.

    ``k_ctx[l][b]`` / ``v_ctx[l][b]``: layer l's cached rows [ctx_b, n_kv,
    head_dim] of sequence b (positions 0..ctx_b-1, as gathered from the pages).
    Returns (logits [B, V], new_k [L, B, n_kv, D], new_v [L, B, n_kv, D],
    hidden [B, H] after the final norm)."""
    p = _params(sd, dtype)
    R = _rounder(mode, dtype)
    tok = torch.as_tensor(token_ids).long().view(-1)
    d, r = None, p["model.embed_tokens.weight"][tok]
    new_k, new_v = [], []
    for i in range(n_layers):
        d, r, k, v = qwen3_decode_layer(sd, i, d, r, positions, k_ctx[i], v_ctx[i], n_heads, n_kv,
                                        head_dim, eps, theta, dtype, mode, p=p)
        new_k.append(k)
        new_v.append(v)
    x = R(_rms(d + r, p["model.norm.weight"], eps))
    head = p.get("lm_head.weight", p["model.embed_tokens.weight"])
    return R(x @ head.T), torch.stack(new_k), torch.stack(new_v), x
