"""Qwen3 model and continuous-batching engine on the gfx950 kernels.

Keeps the call surface of qwen3-naive-inference's qwen3_naive.py so it drops
in under its generator and GRPO loop:
  Qwen3Config / RMSNorm / RotaryEmbedding / Qwen3Attention / Qwen3MLP /
  Qwen3DecoderLayer / Qwen3Model / Qwen3ForCausalLM   (:109-840)
  Qwen3Attention.forward_prefill / forward_decode    (:597-683)
  allocate_global_kv_cache, HIP-graph decode, _prepare_step / _prepare_decode,
  generate_continuous / generate_continuous_with_logprobs (:994-1679)
  store_kvcache (:36) is re-exported from kernels.

Inference paths (no autograd) run the HIP kernels: fused QK-RMSNorm + RoPE,
slot-mapped KV store, paged decode / varlen prefill attention, RMSNorm /
add+RMSNorm, SwiGLU; projections use torch GEMMs (hipBLASLt).  The batch
``forward`` used for training keeps torch ops so autograd works, with a
differentiable RoPE (the reference's RoPE kernel has no backward) and the
attention core in fp32.
"""
from __future__ import annotations

import json
import time
from collections import deque
from dataclasses import dataclass
from functools import lru_cache

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels as K
from .kernels import store_kvcache  # noqa: F401  (reference import surface)
from .paged import (BLOCK_SIZE, BlockManager, Sequence, build_block_tables, fill_decode_inputs,
                    near_equal_contexts, prepare_decode, prepare_step)


@dataclass
class Qwen3Config:
    hidden_size: int = 1024
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    vocab_size: int = 151936
    max_position_embeddings: int = 40960
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000
    attention_bias: bool = False
    hidden_act: str = "silu"
    tie_word_embeddings: bool = True
    bos_token_id: int = 151643
    eos_token_id: int = 151645
    dtype: str = "bfloat16"

    @classmethod
    def from_json(cls, path):
        with open(path, "r") as f:
            d = json.load(f)
        return cls(
            hidden_size=d["hidden_size"], num_attention_heads=d["num_attention_heads"],
            num_key_value_heads=d["num_key_value_heads"],
            head_dim=d.get("head_dim", d["hidden_size"] // d["num_attention_heads"]),
            intermediate_size=d["intermediate_size"], num_hidden_layers=d["num_hidden_layers"],
            vocab_size=d["vocab_size"], max_position_embeddings=d["max_position_embeddings"],
            rms_norm_eps=d["rms_norm_eps"], rope_theta=d.get("rope_theta", 1000000),
            attention_bias=d.get("attention_bias", False), hidden_act=d["hidden_act"],
            tie_word_embeddings=d.get("tie_word_embeddings", True),
            bos_token_id=d.get("bos_token_id", 151643), eos_token_id=d.get("eos_token_id", 151645))


def _use_kernels(*tensors: torch.Tensor) -> bool:
    """HIP kernels serve inference; autograd-tracked calls keep torch ops."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return False
    return all(t.is_cuda for t in tensors)


def _decode_linear(proj: nn.Linear, x: torch.Tensor, parts: bool = False):
    """A decode-step projection: the HIP decode-batch GEMM for bf16 inference
    at <= 256 rows (as fp32 partial products when ``parts``: the residual add
    + RMSNorm that follows sums them), else ``proj(x)``."""
    w = proj.weight
    if proj.bias is None and _use_kernels(x, w) and K.linear_rows_ok(x, w):
        if parts and w.shape[0] <= K.NORM_MAX_WIDTH:  # the norm that sums them takes the width
            return K.linear_rows_parts(x, w)
        return K.linear_rows(x, w)
    return proj(x)


class RMSNorm(nn.Module):
    """RMSNorm with optional fused residual add (qwen3_naive.py:150-175)."""

    def __init__(self, hidden_size, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def _torch(self, x, residual):
        dt = x.dtype
        xf = x.float() if residual is None else x.float() + residual.float()
        res = None if residual is None else xf.to(dt)
        y = (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
             * self.weight.float()).to(dt)
        return y if residual is None else (y, res)

    def forward(self, x, residual=None):
        if isinstance(x, K.RowParts):  # a decode projection's split-K partial products
            if residual is None:
                x = x.dense()
            else:
                return K.add_rms_norm_parts(x, residual, self.weight, self.eps)
        if (x.dtype != torch.bfloat16 or x.shape[-1] > K.NORM_MAX_WIDTH
                or not _use_kernels(x, self.weight)):
            return self._torch(x, residual)
        if residual is None:
            return K.rms_norm(x, self.weight, self.eps)
        return K.add_rms_norm(x, residual, self.weight, self.eps)


class RotaryEmbedding(nn.Module):
    """fp32 cos/sin cache [max_position, head_dim] = cat(cos, sin) (qwen3_naive.py:380-410)."""

    def __init__(self, head_dim, max_position, rope_theta):
        super().__init__()
        inv_freq = 1.0 / (rope_theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
        pos = torch.arange(0, max_position, dtype=torch.float)
        freqs = torch.outer(pos, inv_freq)
        self.register_buffer("cos_sin_cache", torch.cat((freqs.cos(), freqs.sin()), dim=-1))

    @staticmethod
    def rotate(x: torch.Tensor, positions: torch.Tensor, cache: torch.Tensor) -> torch.Tensor:
        """Differentiable half-split rotation (fp32 math, cast back)."""
        half = x.shape[-1] // 2
        cs = cache[positions]
        while cs.dim() < x.dim():
            cs = cs.unsqueeze(-2)
        c, s = cs[..., :half], cs[..., half:]
        x1, x2 = x[..., :half].float(), x[..., half:].float()
        return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(x.dtype)

    def forward(self, q, k, positions):
        return (self.rotate(q, positions, self.cos_sin_cache),
                self.rotate(k, positions, self.cos_sin_cache))


@lru_cache(8)
def _rope_cpu(head_dim: int, max_position: int, rope_theta: float) -> RotaryEmbedding:
    return RotaryEmbedding(head_dim, max_position, rope_theta)


def get_rope(head_dim: int, max_position: int, rope_theta: float) -> RotaryEmbedding:
    """One shared cache per parameter set (the reference shares it across layers)."""
    return _rope_cpu(head_dim, max_position, rope_theta)


class Qwen3Attention(nn.Module):
    """GQA attention with QK-norm and RoPE (qwen3_naive.py:413-683)."""

    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.hidden_size = config.hidden_size
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.scale = self.head_dim ** -0.5
        self.eps = config.rms_norm_eps
        self.qkv_proj = nn.Linear(self.hidden_size, self.q_size + 2 * self.kv_size,
                                  bias=config.attention_bias)
        self.o_proj = nn.Linear(self.q_size, self.hidden_size, bias=False)
        self.q_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.k_cache = None
        self.v_cache = None
        # Decode schedule passed to the attention kernel: 0 = balanced split
        # with merge, -1 = one whole (sequence, head group) unit per
        # workgroup and no merge (the engine picks it for near-equal contexts).
        self.decode_pages_per_split = 0
        # Decode steps fold the QK-norm / RoPE / KV store into the attention
        # launch (qmi_paged_decode_attention_qkv); False runs them as the
        # separate fused norm kernel before the attention.
        self.decode_fused_qkv = True
        # Not a registered submodule: the cache is shared between layers.
        self.__dict__["rotary_emb"] = get_rope(self.head_dim, config.max_position_embeddings,
                                               config.rope_theta)

    def _cos_sin(self, device) -> torch.Tensor:
        rope = self.rotary_emb
        if rope.cos_sin_cache.device != device:
            rope.cos_sin_cache = rope.cos_sin_cache.to(device)
        return rope.cos_sin_cache

    def _project(self, x, positions):
        """qkv projection + fused QK-norm/RoPE kernel -> q [N,Hq,D], k [N,Hkv,D], v view."""
        qkv = self.qkv_proj(x)
        q, k = K.qk_norm_rope(qkv, self.q_norm.weight, self.k_norm.weight, positions,
                              self._cos_sin(x.device), self.num_heads, self.num_kv_heads,
                              self.eps)
        v = qkv[:, self.q_size + self.kv_size:].view(x.shape[0], self.num_kv_heads, self.head_dim)
        return q, k, v

    def _project_store(self, x, positions, slots, decode=False):
        """qkv projection + fused QK-norm/RoPE/KV-store kernel -> q [N,Hq,D]; the
        rotated k and v land in the cache rows ``slots``."""
        qkv = _decode_linear(self.qkv_proj, x) if decode else self.qkv_proj(x)
        return K.qk_norm_rope_store(qkv, self.q_norm.weight, self.k_norm.weight, positions,
                                    self._cos_sin(x.device), self.num_heads, self.num_kv_heads,
                                    self.eps, self.k_cache, self.v_cache, slots)

    # ----- batch path (training / no-cache eager forward, qwen3_naive.py:553-593) -----
    def forward(self, x):
        batch, seq_len, _ = x.shape
        qkv = self.qkv_proj(x)
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = self.q_norm(q.reshape(batch, seq_len, self.num_heads, self.head_dim))
        k = self.k_norm(k.reshape(batch, seq_len, self.num_kv_heads, self.head_dim))
        v = v.reshape(batch, seq_len, self.num_kv_heads, self.head_dim)
        positions = torch.arange(seq_len, device=x.device)
        cache = self._cos_sin(x.device)
        q = RotaryEmbedding.rotate(q, positions[None, :].expand(batch, -1), cache)
        k = RotaryEmbedding.rotate(k, positions[None, :].expand(batch, -1), cache)
        rep = self.num_heads // self.num_kv_heads
        # Attention core in fp32: batched bf16 products with transposed operands
        # (and their autograd) are avoided on this platform.
        qf = q.transpose(1, 2).float()
        kf = k.transpose(1, 2).float().repeat_interleave(rep, dim=1)
        vf = v.transpose(1, 2).float().repeat_interleave(rep, dim=1)
        scores = torch.matmul(qf, kf.transpose(-2, -1).contiguous()) * self.scale
        mask = torch.triu(torch.ones(seq_len, seq_len, device=x.device, dtype=torch.bool), 1)
        scores = scores.masked_fill(mask, float("-inf"))
        w = torch.softmax(scores, dim=-1)
        o = torch.matmul(w, vf).to(x.dtype)
        o = o.transpose(1, 2).reshape(batch, seq_len, -1)
        return self.o_proj(o)

    # ----- continuous batching (qwen3_naive.py:597-683) -----
    def forward_prefill(self, x, positions, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                        max_seqlen_k, block_mapping, block_tables=None):
        """Varlen prefill/mixed step: store the new K/V through ``block_mapping``,
        then attend over the paged cache (prefix + earlier chunks + this chunk)."""
        tokens = x.shape[0]
        q = self._project_store(x, positions, block_mapping)
        o = K.varlen_prefill_attention(q, self.k_cache, self.v_cache, cu_seqlens_q, cu_seqlens_k,
                                       max_seqlen_q, max_seqlen_k, self.scale, True, block_tables)
        return self.o_proj(o.view(tokens, -1))

    def forward_decode(self, x, positions, context_lens, block_tables, slot_mapping=None):
        """One new token per sequence: store its K/V at ``slot_mapping`` (derived
        from the tables when None) and attend over ``context_lens + 1`` keys."""
        batch = x.shape[0]
        if slot_mapping is None:
            ctx = context_lens.long()
            blk = block_tables.long().gather(1, (ctx // BLOCK_SIZE)[:, None])[:, 0]
            slot_mapping = (blk * BLOCK_SIZE + ctx % BLOCK_SIZE).to(torch.int32)
        if (self.decode_fused_qkv and self.decode_pages_per_split <= 0 and _use_kernels(x)
                and K.decode_qkv_ok(self.num_heads, self.num_kv_heads, self.head_dim, batch)):
            qkv = _decode_linear(self.qkv_proj, x)
            o = K.paged_decode_attention_qkv(
                qkv, self.q_norm.weight, self.k_norm.weight, positions, self._cos_sin(x.device),
                self.num_heads, self.num_kv_heads, self.eps, self.k_cache, self.v_cache,
                slot_mapping, context_lens, block_tables, self.scale,
                pages_per_split=self.decode_pages_per_split)
        else:
            q = self._project_store(x, positions, slot_mapping, decode=True)
            o = K.paged_decode_attention(q, self.k_cache, self.v_cache, context_lens,
                                         block_tables, self.scale, seqlen_bias=1,
                                         pages_per_split=self.decode_pages_per_split)
        return _decode_linear(self.o_proj, o.view(batch, -1), parts=True)


class Qwen3MLP(nn.Module):
    """SwiGLU FFN with fused gate/up (qwen3_naive.py:686-702)."""

    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.gate_up_proj = nn.Linear(config.hidden_size, 2 * config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)

    def forward(self, x):
        gu = self.gate_up_proj(x)
        if gu.dtype == torch.bfloat16 and _use_kernels(gu):
            return self.down_proj(K.silu_mul(gu))
        gate, up = gu.chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)

    def forward_decode(self, x):
        """Decode step: gate_up GEMM with the SwiGLU epilogue, then down_proj as
        partial products for the next residual add + RMSNorm (HIP decode-batch
        GEMMs at <= 256 rows; otherwise as ``forward``)."""
        w = self.gate_up_proj.weight
        if (self.gate_up_proj.bias is None and _use_kernels(x, w)
                and K.linear_rows_ok(x, w, swiglu=True)):
            return _decode_linear(self.down_proj, K.linear_rows(x, w, swiglu=True), parts=True)
        return self.forward(x)


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.self_attn = Qwen3Attention(config)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.mlp = Qwen3MLP(config)

    def forward(self, x):
        x = self.self_attn(self.input_layernorm(x)) + x
        return self.mlp(self.post_attention_layernorm(x)) + x

    def forward_prefill(self, x, positions, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                        max_seqlen_k, block_mapping, block_tables=None, residual=None):
        if residual is None:
            h, residual = self.input_layernorm(x), x
        else:
            h, residual = self.input_layernorm(x, residual)
        h = self.self_attn.forward_prefill(h, positions, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                           max_seqlen_k, block_mapping, block_tables)
        h, residual = self.post_attention_layernorm(h, residual)
        return self.mlp(h), residual

    def forward_decode(self, x, positions, context_lens, block_tables, slot_mapping=None,
                       residual=None):
        if residual is None:
            h, residual = self.input_layernorm(x), x
        else:
            h, residual = self.input_layernorm(x, residual)
        h = self.self_attn.forward_decode(h, positions, context_lens, block_tables, slot_mapping)
        h, residual = self.post_attention_layernorm(h, residual)
        return self.mlp.forward_decode(h), residual


class Qwen3Model(nn.Module):
    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([Qwen3DecoderLayer(config)
                                     for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, x):
        h = self.embed_tokens(x)
        for layer in self.layers:
            h = layer(h)
        return self.norm(h)

    def forward_prefill(self, x, positions, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                        max_seqlen_k, block_mapping, block_tables=None):
        h = self.embed_tokens(x)
        residual = None
        for layer in self.layers:
            h, residual = layer.forward_prefill(h, positions, cu_seqlens_q, cu_seqlens_k,
                                                max_seqlen_q, max_seqlen_k, block_mapping,
                                                block_tables, residual)
        h, _ = self.norm(h, residual)
        return h

    def forward_decode(self, x, positions, context_lens, block_tables, slot_mapping=None):
        h = self.embed_tokens(x)
        residual = None
        for layer in self.layers:
            h, residual = layer.forward_decode(h, positions, context_lens, block_tables,
                                               slot_mapping, residual)
        h, _ = self.norm(h, residual)
        return h


# Decode batch sizes captured as HIP graphs.  The reference stops at 64 and
# runs larger batches eagerly; the 288 GB HBM affords buckets up to 256.
GRAPH_BATCH_SIZES = (1, 2, 4, 8, 16, 32, 48, 64, 96, 128, 160, 192, 256)
# Buckets that also get a whole-unit decode graph: from 128 sequences the
# attention's (sequence, head group) units fill two workgroups per CU.
UNIT_GRAPH_MIN_BS = 128
MAX_TOKENS_PER_STEP = 2048
# Stands in for a sampled token whose value is still on the device (decode lookahead).
_PENDING_TOKEN = -1


class Qwen3ForCausalLM(nn.Module):
    """Model + tied lm_head + paged-KV continuous-batching engine."""

    BLOCK_SIZE = BLOCK_SIZE
    packed_modules_mapping = {
        "q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
        "gate_proj": ("gate_up_proj", "gate"), "up_proj": ("gate_up_proj", "up"),
    }

    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.config = config
        self.model = Qwen3Model(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self._num_blocks = 0
        self._graphs: dict = {}
        self._graphs_units: dict = {}
        self._graph_bufs = None
        self._graph_pool = None
        self._has_cuda_graphs = False
        # Launch decode step t+1 before reading step t's tokens back.
        self.decode_lookahead = True
        self._preemptions = 0
        self._preempted: set = set()

    def forward(self, x):
        return self.lm_head(self.model(x))

    # ---------------- KV pool (qwen3_naive.py:994-1066) ----------------
    def kv_block_bytes(self) -> int:
        a = self.model.layers[0].self_attn
        return 2 * len(self.model.layers) * self.BLOCK_SIZE * a.num_kv_heads * a.head_dim * 2

    def _compute_num_blocks(self, gpu_memory_utilization=0.9, warmup_tokens=2048):
        """Blocks that fit in ``utilization * total`` after weights and the peak
        activation of a ``warmup_tokens`` forward (qwen3_naive.py:996-1035)."""
        dev = next(self.parameters()).device
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(dev)
        with torch.no_grad():
            ids = torch.randint(0, self.config.vocab_size, (1, warmup_tokens), device=dev)
            _ = self.forward(ids)
        del _
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        free, total = torch.cuda.mem_get_info(dev)
        stats = torch.cuda.memory_stats(dev)
        peak_act = stats["allocated_bytes.all.peak"] - stats["allocated_bytes.all.current"]
        avail = int(total * gpu_memory_utilization - (total - free) - peak_act)
        return max(avail // self.kv_block_bytes(), 1)

    def allocate_global_kv_cache(self, num_blocks: int | None = None):
        """One [layers, blocks, 256, Hkv, D] bf16 pool for K and one for V; each
        layer gets its slice (qwen3_naive.py:1037-1066).  ``num_blocks`` (or a
        preset ``_num_blocks``) skips the warm-up sizing."""
        if num_blocks:
            self._num_blocks = int(num_blocks)
        if not self._num_blocks:
            self._num_blocks = self._compute_num_blocks()
        a0 = self.model.layers[0].self_attn
        shape = (self._num_blocks, self.BLOCK_SIZE, a0.num_kv_heads, a0.head_dim)
        if a0.k_cache is not None and tuple(a0.k_cache.shape) == shape:
            return
        dev = next(self.parameters()).device
        n = len(self.model.layers)
        for layer in self.model.layers:
            layer.self_attn.k_cache = layer.self_attn.v_cache = None
        self._graphs.clear()
        self._graphs_units.clear()
        self._has_cuda_graphs = False
        torch.cuda.empty_cache()
        k = torch.empty((n,) + shape, dtype=torch.bfloat16, device=dev)
        v = torch.empty((n,) + shape, dtype=torch.bfloat16, device=dev)
        for i, layer in enumerate(self.model.layers):
            layer.self_attn.k_cache = k[i]
            layer.self_attn.v_cache = v[i]

    # ---------------- HIP-graph decode (qwen3_naive.py:1068-1145) ----------------
    def _init_cuda_graphs(self, max_bs: int = GRAPH_BATCH_SIZES[-1], bt_width: int | None = None):
        dev = next(self.parameters()).device
        full = min(self._num_blocks, -(-self.config.max_position_embeddings // self.BLOCK_SIZE))
        bt_width = full if bt_width is None else min(bt_width, full)
        # Every decode input in one int32 device buffer, field after field
        # (ids and positions as int64 pairs, then slots, context lengths and
        # the page tables), so a step's inputs arrive in one host-to-device copy.
        self._graph_in = torch.zeros(6 * max_bs + max_bs * bt_width, dtype=torch.int32, device=dev)
        self._graph_max_bs = max_bs
        v = self._graph_in
        self._graph_bufs = {
            "input_ids": v[0:2 * max_bs].view(torch.long),
            "positions": v[2 * max_bs:4 * max_bs].view(torch.long),
            "slot_mapping": v[4 * max_bs:5 * max_bs],
            "context_lens": v[5 * max_bs:6 * max_bs],
            "block_tables": v[6 * max_bs:].view(max_bs, bt_width),
            "outputs": torch.zeros(max_bs, self.config.hidden_size, dtype=torch.bfloat16,
                                   device=dev),
        }
        self._graph_bufs["slot_mapping"].fill_(-1)
        self._graph_bufs["block_tables"].fill_(-1)
        self._graphs = {}
        self._graphs_units = {}
        self._graph_pool = None
        self._has_cuda_graphs = False

    def _set_decode_schedule(self, pages_per_split: int) -> None:
        for layer in self.model.layers:
            layer.self_attn.decode_pages_per_split = pages_per_split

    def _capture_decode_graphs(self, batch_sizes=GRAPH_BATCH_SIZES):
        """Capture forward_decode for each bucket into one shared memory pool.
        Padded rows carry slot -1 and an empty context, so replays never write
        stale slots.  Buckets of 128 and more get a second graph with the
        whole-unit attention schedule (no merge launches), replayed when the
        step's contexts are near-equal.  Capture failure falls back to eager
        decode."""
        bufs = self._graph_bufs
        max_bs = bufs["input_ids"].shape[0]
        sizes = sorted((b for b in batch_sizes if b <= max_bs), reverse=True)
        plan = [(bs, 0) for bs in sizes] + [(bs, -1) for bs in sizes if bs >= UNIT_GRAPH_MIN_BS]
        try:
            with torch.no_grad():
                for bs, pps in plan:
                    self._set_decode_schedule(pps)
                    args = (bufs["input_ids"][:bs], bufs["positions"][:bs],
                            bufs["context_lens"][:bs], bufs["block_tables"][:bs],
                            bufs["slot_mapping"][:bs])
                    s = torch.cuda.Stream()
                    s.wait_stream(torch.cuda.current_stream())
                    with torch.cuda.stream(s):
                        self.model.forward_decode(*args)
                    torch.cuda.current_stream().wait_stream(s)
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, pool=self._graph_pool):
                        bufs["outputs"][:bs] = self.model.forward_decode(*args)
                    if self._graph_pool is None:
                        self._graph_pool = graph.pool()
                    (self._graphs_units if pps else self._graphs)[bs] = graph
            self._has_cuda_graphs = True
        except Exception as e:
            print(f"HIP graph capture failed, decoding eagerly: {e}")
            self._graphs = {}
            self._graphs_units = {}
            self._has_cuda_graphs = False
        finally:
            self._set_decode_schedule(0)

    def _run_decode_graph(self, bs, input_ids, positions, context_lens, block_tables,
                          slot_mapping):
        graph_bs = next((b for b in sorted(self._graphs) if b >= bs), None)
        bufs = self._graph_bufs
        if graph_bs is None or block_tables.shape[1] > bufs["block_tables"].shape[1]:
            return None
        bufs["input_ids"][:bs] = input_ids
        bufs["positions"][:bs] = positions
        bufs["slot_mapping"][:bs] = slot_mapping
        bufs["slot_mapping"][bs:graph_bs] = -1
        bufs["context_lens"][:bs] = context_lens
        bufs["context_lens"][bs:graph_bs] = 0
        bufs["block_tables"][:bs, :block_tables.shape[1]] = block_tables
        bufs["block_tables"][:bs, block_tables.shape[1]:] = -1
        self._graphs[graph_bs].replay()
        return bufs["outputs"][:bs]

    def _run_decode_graph_seqs(self, seqs, ids_dev=None):
        """Graph decode step straight from the sequences: the inputs of the
        bucket's rows (padding rows: slot -1, empty context, -1 tables) are
        written into a pinned host image of the input buffer and sent in one
        copy; ``ids_dev`` (device token ids, e.g. the previous step's samples)
        replaces the host ids.  Returns None when no captured graph fits."""
        bs = len(seqs)
        graph_bs = next((b for b in sorted(self._graphs) if b >= bs), None)
        bufs = self._graph_bufs
        width = bufs["block_tables"].shape[1]
        if graph_bs is None or max(len(s.block_table) for s in seqs) > width:
            return None
        mb = self._graph_max_bs
        host = torch.empty(self._graph_in.numel(), dtype=torch.int32, pin_memory=True)
        a = host.numpy()
        ids, pos = a[0:2 * mb].view(np.int64), a[2 * mb:4 * mb].view(np.int64)
        slot, ctx = a[4 * mb:5 * mb], a[5 * mb:6 * mb]
        tables = a[6 * mb:].reshape(mb, width)
        fill_decode_inputs(seqs, ids, pos, ctx, slot, tables, self.BLOCK_SIZE)
        ids[bs:graph_bs] = 0
        pos[bs:graph_bs] = 0
        slot[bs:graph_bs] = -1
        ctx[bs:graph_bs] = 0
        tables[bs:graph_bs] = -1
        self._graph_in.copy_(host, non_blocking=True)
        if ids_dev is not None:
            bufs["input_ids"][:bs].copy_(ids_dev)
        graph = self._graphs_units.get(graph_bs) if near_equal_contexts(ctx[:graph_bs]) else None
        if graph is not None and isinstance(getattr(self, "last_stats", None), dict):
            self.last_stats["unit_graph_steps"] = self.last_stats.get("unit_graph_steps", 0) + 1
        (graph or self._graphs[graph_bs]).replay()
        return bufs["outputs"][:bs]

    # ---------------- step preparation (qwen3_naive.py:1147-1225) ----------------
    def _device(self):
        return next(self.parameters()).device

    def _prepare_step(self, seqs):
        return prepare_step(seqs, self._device(), self.BLOCK_SIZE)

    def _build_block_tables(self, seqs):
        t = torch.from_numpy(build_block_tables(seqs))
        return t.pin_memory().to(self._device(), non_blocking=True)

    def _prepare_decode(self, seqs):
        return prepare_decode(seqs, self._device(), self.BLOCK_SIZE)

    # ---------------- generation (qwen3_naive.py:1227-1679) ----------------
    def _ensure_engine(self, graphs: bool, bt_width: int | None = None):
        """KV pool, then decode graphs whose table width covers ``bt_width`` pages."""
        self.allocate_global_kv_cache()
        if not graphs:
            return
        have = self._graph_bufs["block_tables"].shape[1] if self._graph_bufs else 0
        if not self._has_cuda_graphs or (bt_width is not None and have < bt_width):
            self._init_cuda_graphs(bt_width=bt_width)
            self._capture_decode_graphs()

    def _schedule(self, waiting, running, bm):
        """One scheduling round: decode-first walk of ``running`` with LIFO
        preemption, then admission of ``waiting`` with chunked prefill under a
        2048-token budget (qwen3_naive.py:1257-1341)."""
        scheduled = []
        budget = MAX_TOKENS_PER_STEP
        i = 0
        while i < len(running) and budget > 0:
            seq = running[i]
            if seq.kv_len >= seq.num_prompt_tokens:
                if seq.num_completion_tokens >= seq.max_tokens:
                    seq.status = "FINISHED"
                    bm.deallocate(seq.block_table)
                    seq.block_table.clear()
                    running.pop(i)
                    continue
                if seq.kv_len % self.BLOCK_SIZE == 0 and not bm.free:
                    while not bm.can_append(seq):
                        victim = running[-1]
                        victim.status = "WAITING"
                        bm.deallocate(victim.block_table)
                        victim.block_table.clear()
                        victim.kv_len = 0
                        victim.token_ids = victim.token_ids[:victim.num_prompt_tokens]
                        victim.last_token = victim.token_ids[-1]
                        victim.response_log_probs.clear()
                        running.pop()
                        waiting.appendleft(victim)
                        self._preemptions += 1
                        self._preempted.add(getattr(victim, "seq_index", -1))
                        if victim is seq:
                            break
                    if seq.status == "WAITING":
                        continue
                bm.may_append(seq)
                seq.num_scheduled_tokens = 1
            else:
                seq.num_scheduled_tokens = min(seq.num_prompt_tokens - seq.kv_len, budget)
            scheduled.append(seq)
            budget -= seq.num_scheduled_tokens
            i += 1
        while waiting and budget > 0:
            seq = waiting[0]
            if not seq.block_table:
                if bm.available < seq.num_blocks:
                    break
                bm.allocate(seq)
            waiting.popleft()
            seq.status = "RUNNING"
            running.append(seq)
            remaining = seq.num_prompt_tokens - seq.kv_len
            if remaining <= budget:
                seq.num_scheduled_tokens = remaining
            elif not scheduled:
                seq.num_scheduled_tokens = budget
            else:
                waiting.appendleft(seq)
                running.pop()
                break
            scheduled.append(seq)
            budget -= seq.num_scheduled_tokens
        return scheduled

    def _sample(self, h, temperature, top_k, want_logprobs, row_counters=None, seed=None):
        """lm_head + temperature / top-k / softmax / multinomial (qwen3_naive.py:1387,
        :1413-1423) and, optionally, the sampled tokens' log-probabilities
        (:1649-1650), from the final hidden states ``h`` of the sampled rows.

        The fused HIP kernel rounds the logits to bf16 as the reference's
        lm_head output, keeps them out of memory, and draws each token by
        inverse transform sampling with one Philox uniform per row, from all
        entries (top_k None) or from the top k (k <= 64, the reference default
        20); ``row_counters`` (int64 per row) key each row's uniform, else the
        row index does.  Larger k samples from materialised bf16 logits with a
        HIP radix-select sampler."""
        w = self.lm_head.weight
        if top_k is not None and top_k >= w.shape[0]:
            top_k = None  # keeping every entry is plain sampling
        kern = h.dtype == torch.bfloat16 and h.is_cuda and w.dtype == torch.bfloat16
        if kern and (top_k is None or (top_k <= K.MAX_FUSED_TOP_K
                                       and w.shape[0] <= K.MAX_FUSED_TOP_K_VOCAB)):
            return K.lm_head_sample(h, w, temperature, seed=seed, want_logprobs=want_logprobs,
                                    top_k=top_k, row_counters=row_counters)
        if kern and top_k <= 1024:
            return K.sample_tokens_topk(self.lm_head(h), top_k, temperature, seed=seed,
                                        want_logprobs=want_logprobs)
        x = self.lm_head(h).float()
        if temperature != 1.0:
            x = x / temperature
        if top_k is not None:
            vals, idx = torch.topk(x, top_k, dim=-1)
            x = torch.full_like(x, float("-inf")).scatter(-1, idx, vals)
        nxt = torch.multinomial(torch.softmax(x, dim=-1), num_samples=1)
        lp = torch.log_softmax(x, dim=-1).gather(-1, nxt)[:, 0] if want_logprobs else None
        return nxt[:, 0], lp

    def _row_counters(self, seqs):
        """Per-row Philox counter values (j << 32) | i for the j-th generated
        token of the call's i-th sequence: a token's random number depends on
        the call's seed, its sequence and its position only, not on the batch
        it is sampled in (lookahead, preemption and EOS retirement leave the
        draws of the other sequences unchanged)."""
        q = np.fromiter(((s.num_completion_tokens << 32) | s.seq_index for s in seqs),
                        dtype=np.int64, count=len(seqs))
        host = torch.from_numpy(q).pin_memory()
        return host.to(self._device(), non_blocking=True)

    @torch.no_grad()
    def _generate(self, prompt_ids_list, max_new_tokens, temperature, top_k, eos_token_ids,
                  with_logprobs, use_graphs=True):
        eos = set(eos_token_ids) if eos_token_ids is not None else None
        prompts = [p[0].tolist() if torch.is_tensor(p) and p.dim() == 2 else
                   (p.tolist() if torch.is_tensor(p) else list(p)) for p in prompt_ids_list]
        # Graph table width: the pages the longest sequence of this call can need.
        width = -(-(max(len(p) for p in prompts) + max_new_tokens + 1) // self.BLOCK_SIZE)
        self._ensure_engine(use_graphs, bt_width=width)
        bm = BlockManager(self._num_blocks, self.BLOCK_SIZE)
        waiting = deque(Sequence(p, {"temperature": temperature, "max_tokens": max_new_tokens})
                        for p in prompts)
        all_seqs = list(waiting)
        for i, s in enumerate(all_seqs):
            s.seq_index = i
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())  # one per call (torch.manual_seed)
        running: list[Sequence] = []
        self._preemptions = 0
        self._preempted = set()
        self.last_stats = {"steps": 0, "decode_steps": 0, "graph_steps": 0, "unit_graph_steps": 0,
                           "lookahead_steps": 0, "eos_finished": 0, "discarded_rows": 0}
        dev = self._device()
        # Decode lookahead: the host launches decode step t+1 (its input ids
        # gathered on the device from step t's samples) before it reads step
        # t's tokens back; step t's tokens then fill placeholders while step
        # t+1 runs.  A sequence that drew an EOS token at step t is retired
        # when the tokens arrive: its row of step t+1 is discarded (its token
        # dropped, its pages freed; the next step is ordered after it on the
        # stream).
        lookahead = self.decode_lookahead
        pending = None

        def finish(s):
            s.status = "FINISHED"
            bm.deallocate(s.block_table)
            s.block_table.clear()
            if s in running:
                running.remove(s)

        def flush():
            nonlocal pending
            if pending is None:
                return
            pending["event"].synchronize()
            toks = pending["tok_host"].tolist()
            lps = pending["lp_host"].tolist() if pending["lp_host"] is not None else None
            for j, (s, at) in enumerate(pending["seqs"]):
                if at is None or at >= len(s.token_ids) or s.token_ids[at] != _PENDING_TOKEN:
                    continue  # retired, or preempted since (its tokens were rolled back)
                s.token_ids[at] = toks[j]
                if at == len(s.token_ids) - 1:
                    s.last_token = toks[j]
                if lps is not None:
                    s.response_log_probs.append(lps[j])
                if eos is not None and toks[j] in eos and s.status != "FINISHED":
                    self.last_stats["eos_finished"] += 1
                    finish(s)
            pending = None

        while waiting or running:
            scheduled = self._schedule(waiting, running, bm)
            if not scheduled:
                continue
            all_decode = all(s.num_scheduled_tokens == 1 for s in scheduled)
            self.last_stats["steps"] += 1
            if all_decode and lookahead:
                ids_dev = None
                if pending is not None:
                    # A row takes its input id from the previous step's samples
                    # only while its last token is still that placeholder: a
                    # sequence preempted and re-admitted in the same round (a
                    # one-token prefill remainder) was rolled back to its prompt
                    # and must be fed its last prompt token from the host.
                    rows = pending["row_of"]
                    idx = [rows.get(id(s), -1) if s.last_token == _PENDING_TOKEN else -1
                           for s in scheduled]
                    if min(idx) < 0:
                        flush()
                        scheduled = self._drop_finished(scheduled)
                        if not scheduled:
                            continue
                    elif idx == list(range(pending["n"])):
                        ids_dev = pending["tok_dev"]
                    else:
                        ids_dev = pending["tok_dev"][torch.tensor(idx, device=dev)]
                self.last_stats["decode_steps"] += 1
                if ids_dev is not None:
                    self.last_stats["lookahead_steps"] += 1
                rc = self._row_counters(scheduled)
                h = None
                if use_graphs and self._has_cuda_graphs:
                    h = self._run_decode_graph_seqs(scheduled, ids_dev)
                    if h is not None:
                        self.last_stats["graph_steps"] += 1
                if h is None:
                    ids, pos, ctx, bt, slots = self._prepare_decode(scheduled)
                    if ids_dev is not None:
                        ids = ids_dev
                    h = self.model.forward_decode(ids, pos, ctx, bt, slots)
                nxt, lp = self._sample(h, temperature, top_k, with_logprobs, rc, seed)
                n = len(scheduled)
                tok_host = torch.empty((n,), dtype=torch.int64, pin_memory=True)
                tok_host.copy_(nxt, non_blocking=True)
                lp_host = None
                if lp is not None:
                    lp_host = torch.empty((n,), dtype=torch.float32, pin_memory=True)
                    lp_host.copy_(lp, non_blocking=True)
                event = torch.cuda.Event()
                event.record()
                flush()  # the previous step's tokens, while this step runs
                rows_at = []
                for s in scheduled:
                    s.num_scheduled_tokens = 0
                    if s.status == "FINISHED":  # drew EOS last step: this row is discarded
                        self.last_stats["discarded_rows"] += 1
                        rows_at.append((s, None))
                        continue
                    s.kv_len += 1
                    s.append_token(_PENDING_TOKEN)
                    rows_at.append((s, len(s.token_ids) - 1))
                pending = {"seqs": rows_at, "row_of": {id(s): j for j, s in enumerate(scheduled)},
                           "n": n, "tok_dev": nxt, "tok_host": tok_host, "lp_host": lp_host,
                           "event": event}
                for s in scheduled:
                    if s.status != "FINISHED" and s.num_completion_tokens >= s.max_tokens:
                        finish(s)
                continue
            if pending is not None:
                flush()
                scheduled = self._drop_finished(scheduled)
                if not scheduled:
                    continue
                all_decode = all(s.num_scheduled_tokens == 1 for s in scheduled)
            if all_decode:
                self.last_stats["decode_steps"] += 1
                h = None
                if use_graphs and self._has_cuda_graphs:
                    h = self._run_decode_graph_seqs(scheduled)
                    if h is not None:
                        self.last_stats["graph_steps"] += 1
                if h is None:
                    ids, pos, ctx, bt, slots = self._prepare_decode(scheduled)
                    h = self.model.forward_decode(ids, pos, ctx, bt, slots)
                sample_idx = None
            else:
                ids, pos, cu_q, cu_k, mq, mk, bmap, bt = self._prepare_step(scheduled)
                h = self.model.forward_prefill(ids, pos, cu_q, cu_k, mq, mk, bmap, bt)
                sample_idx, off = [], 0
                for s in scheduled:
                    if s.num_scheduled_tokens == 1 or s.kv_len + s.num_scheduled_tokens >= s.num_prompt_tokens:
                        sample_idx.append(off + s.num_scheduled_tokens - 1)
                    off += s.num_scheduled_tokens
            for s in scheduled:
                s.kv_len += s.num_scheduled_tokens
                if not all_decode:
                    bm.hash_blocks(s)
            if sample_idx is not None and not sample_idx:
                for s in scheduled:
                    s.num_scheduled_tokens = 0
                continue
            hs = h if sample_idx is None else h[torch.tensor(sample_idx, device=h.device)]
            sampled = [s for s in scheduled if s.num_scheduled_tokens == 1 or s.kv_len >= s.num_prompt_tokens]
            nxt, lp = self._sample(hs, temperature, top_k, with_logprobs,
                                   self._row_counters(sampled), seed)
            toks = nxt.tolist()
            lps = lp.tolist() if lp is not None else None
            for j, s in enumerate(sampled):
                tok = toks[j]
                s.append_token(tok)
                if lps is not None:
                    s.response_log_probs.append(lps[j])
                if eos is not None and tok in eos:
                    self.last_stats["eos_finished"] += 1
                    finish(s)
                elif s.num_completion_tokens >= s.max_tokens:
                    finish(s)
            for s in scheduled:
                s.num_scheduled_tokens = 0
        flush()
        self.last_stats["preemptions"] = self._preemptions
        self.last_stats["preempted_seqs"] = sorted(self._preempted)
        self.last_stats["blocks_in_use"] = self._num_blocks - bm.available
        return all_seqs

    @staticmethod
    def _drop_finished(scheduled):
        """The scheduled sequences minus those an EOS token just retired."""
        out = []
        for s in scheduled:
            if s.status == "FINISHED":
                s.num_scheduled_tokens = 0
            else:
                out.append(s)
        return out

    def generate_continuous(self, prompt_ids_list, max_new_tokens=256, temperature=0.6, top_k=20,
                            eos_token_ids=None, use_graphs=True):
        """Continuous batching with chunked prefill; returns (token ids, generated ids)."""
        seqs = self._generate(prompt_ids_list, max_new_tokens, temperature, top_k, eos_token_ids,
                              False, use_graphs)
        return [s.token_ids for s in seqs], [s.token_ids[s.num_prompt_tokens:] for s in seqs]

    def generate_continuous_with_logprobs(self, prompt_ids_list, max_new_tokens=256,
                                          temperature=0.6, top_k=20, eos_token_ids=None,
                                          use_graphs=True):
        """As generate_continuous, also returning each sampled token's log-probability
        under the sampling distribution and the prompt lengths."""
        seqs = self._generate(prompt_ids_list, max_new_tokens, temperature, top_k, eos_token_ids,
                              True, use_graphs)
        return ([s.token_ids for s in seqs], [s.token_ids[s.num_prompt_tokens:] for s in seqs],
                [list(s.response_log_probs) for s in seqs], [s.num_prompt_tokens for s in seqs])


def load_weights(model: Qwen3ForCausalLM, checkpoint_path: str) -> None:
    """Load a Qwen3 safetensors checkpoint, packing q/k/v and gate/up into the
    fused projections (qwen3_naive.py:1682-1730); ``lm_head.weight`` is tied."""
    from safetensors import safe_open
    packed = model.packed_modules_mapping
    with safe_open(checkpoint_path, framework="pt", device="cpu") as f:
        for name in f.keys():
            if name == "lm_head.weight":
                continue
            t = f.get_tensor(name)
            for key, (fused, shard) in packed.items():
                if key in name:
                    p = model.get_parameter(name.replace(key, fused))
                    if shard in ("q", "gate"):
                        off = 0
                    elif shard == "k":
                        off = p.shape[0] - 2 * t.shape[0]
                    else:
                        off = p.shape[0] - t.shape[0]
                    p.data[off:off + t.shape[0]] = t.to(p.device, p.dtype)
                    break
            else:
                model.get_parameter(name).data.copy_(t.to(model.get_parameter(name).device))
