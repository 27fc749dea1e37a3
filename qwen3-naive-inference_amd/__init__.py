"""MI355X-native (gfx950) GRPO rollout-and-loss hot path for Qwen3.

Drop-in replacements, behind the reference's own Python call surface, for:
  store_kvcache                      -> kernels.store_kvcache (HIP slot-mapped store)
  Qwen3Attention.forward_decode      -> HIP paged GQA decode attention
  Qwen3Attention.forward_prefill     -> HIP varlen paged causal prefill (MFMA)
  forward_logprob / advantage / loss -> HIP streaming log-softmax gather + fused loss

The package directory name is not a Python identifier; import it with
``importlib.import_module("qwen3-naive-inference_amd")``.
"""
from . import _lib, kernels  # noqa: F401
from .kernels import store_kvcache  # noqa: F401

__all__ = ["kernels", "store_kvcache"]
