"""RMSNorm, fused add+RMSNorm and RoPE restated on the CPU.

Reference: qwen3_naive.py
  RMSNorm._rms_norm      :156-161  fp32 x * rsqrt(mean(x^2) + eps) * w, cast back
  RMSNorm._add_rms_norm  :163-169  x + residual in fp32; residual := that sum cast back
  RotaryEmbedding        :380-387  cache[pos] = cat(cos(pos*f), sin(pos*f)),
                                    f_i = theta^(-2i/D)
  _apply_rope_kernel     :44-67    half-split pairs (j, j+D/2):
                                    o1 = x1*c - x2*s, o2 = x2*c + x1*s in fp32
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * w.float()).to(x.dtype)


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor, eps: float = 1e-6):
    xf = x.float() + residual.float()
    res = xf.to(x.dtype)
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * w.float()).to(x.dtype), res


def rope_cache(head_dim: int, max_position: int, theta: float) -> torch.Tensor:
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    pos = torch.arange(0, max_position, dtype=torch.float)
    freqs = torch.outer(pos, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def apply_rope(x: torch.Tensor, positions: torch.Tensor, cache: torch.Tensor,
               out_dtype=None) -> torch.Tensor:
    """x [N, H, D] rotated per token by cache[positions[N]] -> out_dtype."""
    out_dtype = out_dtype or x.dtype
    half = x.shape[-1] // 2
    cs = cache[positions.long()]
    c = cs[:, None, :half].float()
    s = cs[:, None, half:].float()
    x1 = x[..., :half].float()
    x2 = x[..., half:].float()
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(out_dtype)


def apply_rope_complex(x: torch.Tensor, positions: torch.Tensor, head_dim: int,
                       theta: float) -> torch.Tensor:
    """Independent textbook form in float64: pair (x_j, x_{j+D/2}) as the complex
    number x_j + i x_{j+D/2}, multiplied by exp(i * pos * theta^(-2j/D))."""
    half = head_dim // 2
    inv = theta ** (-torch.arange(0, half, dtype=torch.float64) * 2 / head_dim)
    ang = positions.double()[:, None] * inv[None, :]
    rot = torch.polar(torch.ones_like(ang), ang)[:, None, :]
    z = torch.complex(x[..., :half].double(), x[..., half:].double()) * rot
    return torch.cat((z.real, z.imag), dim=-1)
