"""MI355X-native (gfx950) GRPO rollout-and-loss hot path for Qwen3.

Drop-in replacements, behind the reference's own Python call surface, for:
  store_kvcache                      -> kernels.store_kvcache (HIP slot-mapped store)
  Qwen3Attention.forward_decode      -> HIP paged GQA decode attention
  Qwen3Attention.forward_prefill     -> HIP varlen paged causal prefill (MFMA)
  forward_logprob / advantage / loss -> HIP streaming log-softmax gather + fused loss

The package directory name is not a Python identifier; import it with
``importlib.import_module("qwen3-naive-inference_amd")``.
"""
from . import _lib, kernels, paged  # noqa: F401
from .kernels import store_kvcache  # noqa: F401
from . import qwen3_naive, qwen3_grpo_train  # noqa: F401
from .paged import BlockManager, Sequence  # noqa: F401
from .qwen3_naive import (  # noqa: F401
    Qwen3Attention, Qwen3Config, Qwen3DecoderLayer, Qwen3ForCausalLM, Qwen3MLP, Qwen3Model,
    RMSNorm, RotaryEmbedding, load_weights)
from .qwen3_grpo_train import (  # noqa: F401
    compute_grpo_advantage, forward_logprob, grpo_fused_loss, grpo_fused_train_step,
    grpo_loss_from_hidden, grpo_train_step, ppo_clipped_loss)

__all__ = [
    "kernels", "paged", "qwen3_naive", "qwen3_grpo_train", "store_kvcache", "BlockManager",
    "Sequence", "Qwen3Attention", "Qwen3Config", "Qwen3DecoderLayer", "Qwen3ForCausalLM",
    "Qwen3MLP", "Qwen3Model", "RMSNorm", "RotaryEmbedding", "load_weights",
    "compute_grpo_advantage", "forward_logprob", "grpo_fused_loss", "grpo_fused_train_step",
    "grpo_loss_from_hidden", "grpo_train_step", "ppo_clipped_loss",
]
