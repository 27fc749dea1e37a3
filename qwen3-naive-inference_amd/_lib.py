"""ctypes binding of ``libqwen3mi.so`` (the C ABI declared in include/qwen3mi.h).

torch is imported first on purpose: the library's HIP runtime dependency then
resolves to the runtime torch already loaded, so torch's streams and device
pointers are valid in the library.  There is no fallback: if the library is
missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "libqwen3mi.so"

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_f32 = ctypes.c_float
_c_p = ctypes.c_void_p

# name -> (restype, argtypes).  Mirrors include/qwen3mi.h.
SIGNATURES: dict[str, tuple] = {
    "qmi_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "qmi_version": (ctypes.c_int, []),
    "qmi_store_kvcache": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64,
                                         _c_i64, _c_i64, _c_p]),
    "qmi_paged_decode_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "qmi_paged_decode_attention": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64,            # q, strides
        _c_p, _c_p, _c_i64, _c_i64,      # caches, num_blocks, block_size
        _c_i64, _c_i64, _c_i64,          # heads, kv heads, head_dim
        _c_p, _c_i32,                    # seqlens, bias
        _c_p, _c_i64, _c_i64,            # block_table, stride, width
        _c_i64, _c_f32,                  # batch, scale
        _c_p, _c_i64, _c_i64,            # out, strides
        _c_p, _c_i64, _c_i64, _c_p]),    # workspace, bytes, pages_per_split, stream
    "qmi_paged_decode_attention_noalloc": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64,            # q, strides
        _c_p, _c_p, _c_i64, _c_i64,      # caches, num_blocks, block_size
        _c_i64, _c_i64, _c_i64,          # heads, kv heads, head_dim
        _c_p, _c_i32,                    # seqlens, bias
        _c_p, _c_i64, _c_i64,            # block_table, stride, width
        _c_i64, _c_f32,                  # batch, scale
        _c_p, _c_i64, _c_i64,            # out, strides
        _c_i64, _c_p]),                  # pages_per_split, stream
    "qmi_paged_decode_attention_qkv": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_i64,    # qkv, stride, heads, kv heads
        _c_i64, _c_p, _c_p,              # head_dim, q_norm / k_norm weights
        _c_p, _c_p, _c_i64, _c_f32,      # positions, cos_sin_cache, max_position, eps
        _c_p, _c_p, _c_i64, _c_i64,      # caches, num_blocks, block_size
        _c_p, _c_p,                      # slot_mapping, seqlens
        _c_p, _c_i64, _c_i64,            # block_table, stride, width
        _c_i64, _c_f32,                  # batch, scale
        _c_p, _c_i64, _c_i64,            # out, strides
        _c_p, _c_i64, _c_i64, _c_p]),    # workspace, bytes, pages_per_split, stream
    "qmi_varlen_prefill_workspace_bytes": (_c_i64, [_c_i64] * 7),
    "qmi_varlen_prefill_attention": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64,            # q, strides
        _c_p, _c_p, _c_i64, _c_i64,      # caches, num_blocks, block_size
        _c_i64, _c_i64, _c_i64,          # heads, kv heads, head_dim
        _c_p, _c_p,                      # cu_seqlens_q / k
        _c_p, _c_i64, _c_i64,            # block_table, stride, width
        _c_i64, _c_i64, _c_i64,          # batch, max_seqlen_q, max_seqlen_k
        _c_i64, _c_f32,                  # total_q, scale
        _c_p, _c_i64, _c_i64,            # out, strides
        _c_p, _c_i64, _c_i64, _c_p]),    # workspace, bytes, split_keys, stream
    "qmi_rms_norm": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_f32,
                                    _c_p]),
    "qmi_add_rms_norm": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p,
                                        _c_i64, _c_i64, _c_i64, _c_f32, _c_p]),
    "qmi_qk_norm_rope": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p,
                                        _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_f32,
                                        _c_p]),
    "qmi_qk_norm_rope_store": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p,
        _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_f32, _c_p]),
    "qmi_silu_mul": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p]),
    "qmi_linear_rows": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32,
                                       _c_p, _c_i64, _c_p]),
    "qmi_linear_rows_parts_count": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "qmi_linear_rows_parts": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
                                             _c_p, _c_i64, _c_p]),
    "qmi_add_rms_norm_parts": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_i64,
                                              _c_p, _c_p, _c_i64, _c_i64, _c_f32, _c_p]),
    "qmi_logprob_gather": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                          _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "qmi_grpo_advantage": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_f32, _c_p, _c_p]),
    "qmi_ppo_clipped_loss": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                            _c_i64, _c_f32, _c_i32, _c_p, _c_p, _c_p]),
    "qmi_grpo_fused_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "qmi_grpo_fused_loss": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_p, _c_p, _c_p, _c_p, _c_f32, _c_f32, _c_i32,
        _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "qmi_logprob_gather_backward": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p]),
    "qmi_sample_tokens_topk": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, ctypes.c_uint64, ctypes.c_uint64, _c_p,
        _c_p, _c_p]),
    "qmi_lm_head_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "qmi_lm_head_sample": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_f32, _c_i64, ctypes.c_uint64,
        ctypes.c_uint64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "qmi_lm_head_logprob": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p,
        _c_i64, _c_p]),
    "qmi_sample_tokens": (ctypes.c_int, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_f32, ctypes.c_uint64, ctypes.c_uint64, _c_p, _c_p, _c_p]),
}

_LIB = None


class QmiError(RuntimeError):
    """A qwen3mi entry point returned a non-zero status."""


def lib():
    """Load (once) and return the configured ctypes library; raises if absent."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise QmiError(
                f"{LIB_PATH} is missing: build it with `python __graft_entry__.py build` "
                "or qwen3-naive-inference_amd/build.py (hipcc, gfx950)")
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().qmi_error_string(status).decode()
        raise QmiError(f"{what} failed ({status}): {msg}")


def stream_handle(device: torch.device | None = None) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream
