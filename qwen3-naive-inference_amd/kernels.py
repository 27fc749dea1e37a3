"""Python shims over the C ABI: validate, then launch on torch's current stream.

Each shim keeps the argument names, order and meaning of the reference call it
replaces.  Validation failures raise ``ValueError`` before anything is
launched; a failed launch raises ``QmiError``.  All outputs and workspaces are
allocated through torch's caching allocator (graph-capture safe); the kernels
never allocate, synchronise or read device data on the host.
"""
from __future__ import annotations

import torch

from ._lib import check, lib, stream_handle

BLOCK_SIZE = 256
HEAD_DIM = 128

REDUCTIONS = {"token": 0, "token_mean": 0, "seq": 1, "seq_mean": 1}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got {t.device})")


def _require_dtype(name: str, t: torch.Tensor, *dtypes: torch.dtype) -> None:
    if t.dtype not in dtypes:
        raise ValueError(f"{name} must have dtype in {dtypes}, got {t.dtype}")


def _as_i32(name: str, t: torch.Tensor) -> torch.Tensor:
    _require_cuda(name, t)
    if t.dtype == torch.int32:
        return t
    if t.dtype in (torch.int64, torch.int16, torch.uint8, torch.int8):
        return t.to(torch.int32)
    raise ValueError(f"{name} must be an integer tensor, got {t.dtype}")


# ---------------------------------------------------------------------------
# KV store (qwen3_naive.py:20-41)
# ---------------------------------------------------------------------------
def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Write ``key[i]`` / ``value[i]`` into cache row ``slot_mapping[i]`` (-1 skips).

    ``key``/``value``: ``[N, kv_heads, head_dim]`` bf16 whose inner
    ``[kv_heads, head_dim]`` block is contiguous (``value`` may be a strided
    view of the fused qkv projection).  ``k_cache``/``v_cache``: contiguous
    paged pools ``[num_blocks, block_size, kv_heads, head_dim]``.
    """
    for n, t in (("key", key), ("value", value), ("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda(n, t)
        _require_dtype(n, t, torch.bfloat16)
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError(f"key/value must be [N, H, D] of equal shape, got {tuple(key.shape)} "
                         f"and {tuple(value.shape)}")
    n_tok, h, d = key.shape
    row = h * d
    for n, t in (("key", key), ("value", value)):
        if t.stride(2) != 1 or t.stride(1) != d:
            raise ValueError(f"{n}'s [heads, head_dim] block must be contiguous")
    for n, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        if not t.is_contiguous() or t.numel() % row != 0:
            raise ValueError(f"{n} must be contiguous with rows of {row} elements")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")
    slots = _as_i32("slot_mapping", slot_mapping)
    if slots.dim() != 1 or slots.shape[0] != n_tok:
        raise ValueError(f"slot_mapping must be [{n_tok}], got {tuple(slots.shape)}")
    if not slots.is_contiguous():
        slots = slots.contiguous()
    if n_tok == 0:
        return
    st = lib().qmi_store_kvcache(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                                 k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(), n_tok,
                                 row, k_cache.numel() // row, stream_handle(key.device))
    check(st, "store_kvcache")


# ---------------------------------------------------------------------------
# Paged decode attention (flash_attn_with_kvcache at qwen3_naive.py:672-680)
# ---------------------------------------------------------------------------
def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           cache_seqlens: torch.Tensor, block_table: torch.Tensor,
                           softmax_scale: float, seqlen_bias: int = 0,
                           out: torch.Tensor | None = None,
                           pages_per_split: int = 0) -> torch.Tensor:
    """GQA attention of one query per sequence over its paged KV.

    ``q``: ``[B, Hq, D]`` bf16 (unit stride along D).  Sequence ``b`` attends
    to keys ``0 .. cache_seqlens[b] + seqlen_bias - 1`` (flash-attn's
    ``cache_seqlens``; ``forward_decode`` passes ``context_lens`` with bias 1).
    Returns ``out`` ``[B, Hq, D]`` bf16.
    """
    for n, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda(n, t)
        _require_dtype(n, t, torch.bfloat16)
    if q.dim() != 3:
        raise ValueError(f"q must be [B, Hq, D], got {tuple(q.shape)}")
    bsz, hq, d = q.shape
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("caches must be [num_blocks, block_size, Hkv, D] of equal shape")
    nb, bs, hkv, dk = k_cache.shape
    if d != HEAD_DIM or dk != HEAD_DIM or bs != BLOCK_SIZE:
        raise ValueError(f"supported: head_dim {HEAD_DIM}, block_size {BLOCK_SIZE}; got "
                         f"q D={d}, cache {tuple(k_cache.shape)}")
    if hq % hkv != 0 or (hq // hkv) not in (1, 2, 4, 8):
        raise ValueError(f"GQA ratio Hq/Hkv must be 1, 2, 4 or 8 (Hq={hq}, Hkv={hkv})")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if q.stride(2) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = _dense16(q)
    seqlens = _as_i32("cache_seqlens", cache_seqlens)
    bt = _as_i32("block_table", block_table)
    if seqlens.dim() != 1 or seqlens.shape[0] != bsz:
        raise ValueError(f"cache_seqlens must be [{bsz}]")
    if not seqlens.is_contiguous():
        seqlens = seqlens.contiguous()
    if bt.dim() != 2 or bt.shape[0] != bsz or bt.shape[1] < 1:
        raise ValueError(f"block_table must be [{bsz}, W>=1], got {tuple(bt.shape)}")
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    if out is None:
        out = torch.empty((bsz, hq, d), dtype=torch.bfloat16, device=q.device)
    else:
        _require_cuda("out", out)
        _require_dtype("out", out, torch.bfloat16)
        if out.shape != (bsz, hq, d) or out.stride(2) != 1:
            raise ValueError("out must be [B, Hq, D] with unit stride along D")
    if bsz == 0:
        return out
    L = lib()
    wbytes = L.qmi_paged_decode_workspace_bytes(bsz, hkv, hq, bt.shape[1], pages_per_split)
    ws = torch.empty((max(wbytes, 4) // 4,), dtype=torch.float32, device=q.device)
    st = L.qmi_paged_decode_attention(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), nb, bs,
        hq, hkv, d, seqlens.data_ptr(), int(seqlen_bias), bt.data_ptr(), bt.stride(0),
        bt.shape[1], bsz, float(softmax_scale), out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), ws.numel() * 4, int(pages_per_split), stream_handle(q.device))
    check(st, "paged_decode_attention")
    return out


def decode_qkv_ok(num_q_heads: int, num_kv_heads: int, head_dim: int, batch: int) -> bool:
    """Whether ``paged_decode_attention_qkv`` takes this layout and batch."""
    return (head_dim == HEAD_DIM and num_kv_heads in (2, 4, 8, 16)
            and num_q_heads % num_kv_heads == 0 and num_q_heads // num_kv_heads in (1, 2, 4)
            and 0 < batch <= 1024)


def paged_decode_attention_qkv(qkv: torch.Tensor, q_norm_weight: torch.Tensor,
                               k_norm_weight: torch.Tensor, positions: torch.Tensor,
                               cos_sin_cache: torch.Tensor, num_q_heads: int, num_kv_heads: int,
                               eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor,
                               slot_mapping: torch.Tensor, cache_seqlens: torch.Tensor,
                               block_table: torch.Tensor, softmax_scale: float,
                               out: torch.Tensor | None = None,
                               pages_per_split: int = 0) -> torch.Tensor:
    """``qk_norm_rope_store`` followed by ``paged_decode_attention(...,
    seqlen_bias=1)`` in one attention launch: the q heads of the packed
    ``qkv [B, (Hq + 2 Hkv) * 128]`` rows are normalised and rotated inside
    the attention kernel, and the new token's rotated k and its v go to cache
    rows ``slot_mapping`` (-1 skips; otherwise the slot of key
    ``cache_seqlens[b]``, which is then read from the new rows).  Returns
    ``out [B, Hq, 128]``.  ``pages_per_split``: 0 (balanced split + merge)
    or -1 (one whole unit per workgroup, no merge launch)."""
    _require_cuda("qkv", qkv)
    _require_dtype("qkv", qkv, torch.bfloat16)
    width = (num_q_heads + 2 * num_kv_heads) * HEAD_DIM
    if qkv.dim() != 2 or qkv.shape[1] != width:
        raise ValueError(f"qkv must be [B, {width}]")
    if qkv.stride(1) != 1 or qkv.stride(0) % 8 or qkv.data_ptr() % 16:
        qkv = _dense16(qkv)
    bsz = qkv.shape[0]
    for n, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda(n, t)
        _require_dtype(n, t, torch.bfloat16)
    if (k_cache.dim() != 4 or k_cache.shape != v_cache.shape or not k_cache.is_contiguous()
            or not v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous [num_blocks, 256, Hkv, 128] of equal shape")
    nb, bs, hkv, dk = k_cache.shape
    if bs != BLOCK_SIZE or dk != HEAD_DIM or hkv != num_kv_heads:
        raise ValueError(f"caches must be [num_blocks, {BLOCK_SIZE}, {num_kv_heads}, {HEAD_DIM}]")
    if pages_per_split not in (0, -1):
        raise ValueError("pages_per_split must be 0 or -1 (balanced schedule)")
    for n, t in (("positions", positions), ("cos_sin_cache", cos_sin_cache),
                 ("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _require_cuda(n, t)
    cache = cos_sin_cache
    if cache.dtype != torch.float32 or cache.dim() != 2 or cache.shape[1] != HEAD_DIM:
        raise ValueError("cos_sin_cache must be fp32 [max_position, 128]")
    cache = _dense16(cache)
    pos = positions.reshape(-1)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    sl = _as_i32("slot_mapping", slot_mapping).reshape(-1)
    seqlens = _as_i32("cache_seqlens", cache_seqlens).reshape(-1)
    if pos.shape[0] != bsz or sl.shape[0] != bsz or seqlens.shape[0] != bsz:
        raise ValueError(f"positions, slot_mapping and cache_seqlens must have {bsz} entries")
    pos, sl, seqlens = pos.contiguous(), sl.contiguous(), seqlens.contiguous()
    bt = _as_i32("block_table", block_table)
    if bt.dim() != 2 or bt.shape[0] != bsz or bt.shape[1] < 1:
        raise ValueError(f"block_table must be [{bsz}, W>=1], got {tuple(bt.shape)}")
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    qw = _dense16(q_norm_weight.to(torch.bfloat16))
    kw = _dense16(k_norm_weight.to(torch.bfloat16))
    if out is None:
        out = torch.empty((bsz, num_q_heads, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    elif out.shape != (bsz, num_q_heads, HEAD_DIM) or out.stride(2) != 1:
        raise ValueError("out must be [B, Hq, 128] with unit stride along the head dim")
    if bsz == 0:
        return out
    L = lib()
    wbytes = L.qmi_paged_decode_workspace_bytes(bsz, num_kv_heads, num_q_heads, bt.shape[1], 0)
    ws = torch.empty((max(wbytes, 4) // 4,), dtype=torch.float32, device=qkv.device)
    check(L.qmi_paged_decode_attention_qkv(
        qkv.data_ptr(), qkv.stride(0), num_q_heads, num_kv_heads, HEAD_DIM, qw.data_ptr(),
        kw.data_ptr(), pos.data_ptr(), cache.data_ptr(), cache.shape[0], float(eps),
        k_cache.data_ptr(), v_cache.data_ptr(), nb, bs, sl.data_ptr(), seqlens.data_ptr(),
        bt.data_ptr(), bt.stride(0), bt.shape[1], bsz, float(softmax_scale), out.data_ptr(),
        out.stride(0), out.stride(1), ws.data_ptr(), ws.numel() * 4, int(pages_per_split),
        stream_handle(qkv.device)), "paged_decode_attention_qkv")
    return out


# ---------------------------------------------------------------------------
# Varlen paged causal prefill (flash_attn_varlen_func at qwen3_naive.py:631-637)
# ---------------------------------------------------------------------------
# Prefill workspaces.  The first bytes of a workspace hold the work-queue
# counters of the attention kernel, which must be zero before a launch and
# are left zero by every launch: a buffer is zero-filled when allocated and
# then reused.  Eager calls reuse one buffer per (device, stream) -- calls on
# one stream run in stream order, calls on two streams never share counters
# -- and a larger problem gets a new buffer (the old one is released in
# stream order by the caching allocator).  Under graph capture every call
# gets a zero-filled buffer of its own from the graph's memory pool: the
# captured fill re-zeroes it on each replay, and no eager call can resize or
# free memory a graph replays into.
_PREFILL_WS: dict[tuple[int, int], torch.Tensor] = {}


def _prefill_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    n = (nbytes + 3) // 4
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(n, dtype=torch.float32, device=device)
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _PREFILL_WS.get(key)
    if ws is None or ws.numel() < n:
        ws = torch.zeros(n, dtype=torch.float32, device=device)
        _PREFILL_WS[key] = ws
    return ws


def varlen_prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                             max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
                             causal: bool = True, block_table: torch.Tensor | None = None,
                             out: torch.Tensor | None = None, *,
                             split_keys: int = 0,
                             workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Varlen causal attention of the new tokens over their paged K/V.

    Argument order and meaning follow the reference call
    ``flash_attn_varlen_func(q, k_cache, v_cache, max_seqlen_q=..., cu_seqlens_q=...,
    max_seqlen_k=..., cu_seqlens_k=..., softmax_scale=..., causal=True,
    block_table=...)``.  ``q``: ``[Tq, Hq, 128]`` bf16; caches
    ``[num_blocks, 256, Hkv, 128]``; ``cu_seqlens_*``: int32 ``[B+1]``;
    ``block_table``: int32 ``[B, W]``.  Returns ``[Tq, Hq, 128]`` bf16.
    The kernel reads the per-sequence key counts from ``cu_seqlens_k``;
    ``max_seqlen_k`` only sizes the split of long key ranges across
    workgroups.  With ``split_keys=0`` the library schedules the launch:
    launches of a few rounds of (query block, sequence, KV head) items run on
    a persistent grid fed by a work queue, thin ones (no more items per KV
    head than workgroups) with their long items split and merged by a
    second kernel, tiny ones (fewer than 256 items) split across workgroups;
    ``split_keys > 0`` forces pieces of that many keys.  ``workspace``
    (float32, at least ``qmi_varlen_prefill_workspace_bytes`` bytes, zeroed
    before its first use and left zeroed by every call) defaults to one
    cached per (device, stream), or a fresh one per call under graph
    capture.
    """
    if not causal:
        raise ValueError("only causal=True is supported (the reference always passes it)")
    if block_table is None:
        raise ValueError("block_table is required: keys are always read from the paged cache")
    for n, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda(n, t)
        _require_dtype(n, t, torch.bfloat16)
    if q.dim() != 3:
        raise ValueError(f"q must be [Tq, Hq, D], got {tuple(q.shape)}")
    tq, hq, d = q.shape
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("caches must be [num_blocks, block_size, Hkv, D] of equal shape")
    nb, bs, hkv, dk = k_cache.shape
    if d != HEAD_DIM or dk != HEAD_DIM or bs != BLOCK_SIZE:
        raise ValueError(f"supported: head_dim {HEAD_DIM}, block_size {BLOCK_SIZE}")
    if hq % hkv != 0 or (hq // hkv) not in (1, 2, 4):
        raise ValueError(f"GQA ratio Hq/Hkv must be 1, 2 or 4 (Hq={hq}, Hkv={hkv})")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if q.stride(2) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = _dense16(q)
    cq = _as_i32("cu_seqlens_q", cu_seqlens_q).contiguous()
    ck = _as_i32("cu_seqlens_k", cu_seqlens_k).contiguous()
    bt = _as_i32("block_table", block_table)
    if cq.dim() != 1 or ck.shape != cq.shape or cq.shape[0] < 1:
        raise ValueError("cu_seqlens_q / cu_seqlens_k must both be [B+1]")
    bsz = cq.shape[0] - 1
    if bt.dim() != 2 or bt.shape[0] != bsz or bt.shape[1] < 1:
        raise ValueError(f"block_table must be [{bsz}, W>=1], got {tuple(bt.shape)}")
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    if out is None:
        out = torch.empty((tq, hq, d), dtype=torch.bfloat16, device=q.device)
    else:
        _require_cuda("out", out)
        _require_dtype("out", out, torch.bfloat16)
        if out.shape != (tq, hq, d) or out.stride(2) != 1:
            raise ValueError("out must be [Tq, Hq, D] with unit stride along D")
    if bsz == 0 or tq == 0 or int(max_seqlen_q) == 0:
        return out
    split_keys = int(split_keys)
    if split_keys < 0 or split_keys % 64:
        raise ValueError(f"split_keys must be 0 or a positive multiple of 64, got {split_keys}")
    ws_bytes = lib().qmi_varlen_prefill_workspace_bytes(
        bsz, int(max_seqlen_q), int(max_seqlen_k), hq, hkv, bt.shape[1], split_keys)
    if workspace is None:
        ws = _prefill_workspace(q.device, ws_bytes) if ws_bytes > 0 else None
    else:
        _require_cuda("workspace", workspace)
        _require_dtype("workspace", workspace, torch.float32)
        if workspace.numel() * 4 < ws_bytes or not workspace.is_contiguous():
            raise ValueError(f"workspace must be contiguous with at least {ws_bytes} bytes")
        ws = workspace
        ws_bytes = workspace.numel() * 4
    st = lib().qmi_varlen_prefill_attention(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), nb, bs,
        hq, hkv, d, cq.data_ptr(), ck.data_ptr(), bt.data_ptr(), bt.stride(0), bt.shape[1], bsz,
        int(max_seqlen_q), int(max_seqlen_k), tq, float(softmax_scale), out.data_ptr(),
        out.stride(0), out.stride(1), _ptr(ws), ws_bytes, split_keys, stream_handle(q.device))
    check(st, "varlen_prefill_attention")
    return out


# ---------------------------------------------------------------------------
# RMSNorm / QK-norm + RoPE / SwiGLU (qwen3_naive.py:44-80, :156-169, :695-702)
# ---------------------------------------------------------------------------
def _dense16(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself if contiguous and 16-byte aligned, else a contiguous copy
    (a fresh allocation is aligned; ``contiguous()`` alone does not copy a
    contiguous view that starts mid-row)."""
    if not t.is_contiguous():
        return t.contiguous()
    return t.clone() if t.data_ptr() % 16 else t


def _rows2d(name: str, x: torch.Tensor) -> torch.Tensor:
    _require_cuda(name, x)
    _require_dtype(name, x, torch.bfloat16)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = _dense16(x2)
    return x2


NORM_MAX_WIDTH = 4096  # widest row the RMSNorm kernels take (128 lanes x 4 x 8 bf16)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``bf16(x * rsqrt(mean(x^2) + eps) * w)`` over the last dim (fp32 math)."""
    x2 = _rows2d("x", x)
    w = weight.to(torch.bfloat16).contiguous()
    y = torch.empty(x2.shape, dtype=torch.bfloat16, device=x2.device)
    check(lib().qmi_rms_norm(x2.data_ptr(), x2.stride(0), w.data_ptr(), y.data_ptr(), y.stride(0),
                             x2.shape[0], x2.shape[1], float(eps), stream_handle(x2.device)),
          "rms_norm")
    return y.view(x.shape)


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """``s = x + residual``; returns ``(rms_norm(s), bf16(s))`` (fused)."""
    x2 = _rows2d("x", x)
    r2 = _rows2d("residual", residual)
    if r2.shape != x2.shape:
        raise ValueError("x and residual must have the same shape")
    w = weight.to(torch.bfloat16).contiguous()
    y = torch.empty(x2.shape, dtype=torch.bfloat16, device=x2.device)
    r_out = torch.empty_like(y)
    check(lib().qmi_add_rms_norm(x2.data_ptr(), x2.stride(0), r2.data_ptr(), r2.stride(0),
                                 r_out.data_ptr(), r_out.stride(0), w.data_ptr(), y.data_ptr(),
                                 y.stride(0), x2.shape[0], x2.shape[1], float(eps),
                                 stream_handle(x2.device)),
          "add_rms_norm")
    return y.view(x.shape), r_out.view(x.shape)


def qk_norm_rope(qkv: torch.Tensor, q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
                 positions: torch.Tensor, cos_sin_cache: torch.Tensor, num_q_heads: int,
                 num_kv_heads: int, eps: float):
    """Per-head RMSNorm of q and k followed by half-split RoPE, from fused qkv rows.

    ``qkv``: ``[N, (Hq + 2 Hkv) * 128]`` bf16.  Returns contiguous
    ``q [N, Hq, 128]`` and ``k [N, Hkv, 128]``; v stays a view of ``qkv``.
    """
    _require_cuda("qkv", qkv)
    _require_dtype("qkv", qkv, torch.bfloat16)
    if qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a row-major [N, (Hq + 2 Hkv) * 128] tensor")
    if qkv.data_ptr() % 16 or qkv.stride(0) % 8:
        qkv = _dense16(qkv)  # the kernel reads rows 8 / 16 bytes at a time
    n = qkv.shape[0]
    for nm, t in (("positions", positions), ("cos_sin_cache", cos_sin_cache),
                  ("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _require_cuda(nm, t)
    pos = positions.reshape(-1)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    if pos.shape[0] != n:
        raise ValueError(f"positions must have {n} entries")
    pos = pos.contiguous()
    cache = cos_sin_cache
    if cache.dtype != torch.float32 or cache.dim() != 2 or cache.shape[1] != HEAD_DIM:
        raise ValueError("cos_sin_cache must be fp32 [max_position, 128]")
    cache = cache.contiguous()
    qw = q_norm_weight.to(torch.bfloat16).contiguous()
    kw = k_norm_weight.to(torch.bfloat16).contiguous()
    q = torch.empty((n, num_q_heads, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    k = torch.empty((n, num_kv_heads, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    check(lib().qmi_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), n, num_q_heads, num_kv_heads,
                                 HEAD_DIM, qw.data_ptr(), kw.data_ptr(), pos.data_ptr(),
                                 cache.data_ptr(), cache.shape[0], q.data_ptr(), q.stride(0),
                                 k.data_ptr(), k.stride(0), float(eps), stream_handle(qkv.device)),
          "qk_norm_rope")
    return q, k


def qk_norm_rope_store(qkv: torch.Tensor, q_norm_weight: torch.Tensor,
                       k_norm_weight: torch.Tensor, positions: torch.Tensor,
                       cos_sin_cache: torch.Tensor, num_q_heads: int, num_kv_heads: int,
                       eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       slot_mapping: torch.Tensor) -> torch.Tensor:
    """``qk_norm_rope`` with the KV store fused in: returns ``q [N, Hq, 128]`` and
    writes the rotated k and the v heads of ``qkv`` to cache rows ``slot_mapping``
    (-1 skips), bit-identical to ``qk_norm_rope`` + ``store_kvcache``."""
    _require_cuda("qkv", qkv)
    _require_dtype("qkv", qkv, torch.bfloat16)
    if qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a row-major [N, (Hq + 2 Hkv) * 128] tensor")
    if qkv.data_ptr() % 16 or qkv.stride(0) % 8:
        qkv = _dense16(qkv)  # the kernel reads rows 8 / 16 bytes at a time
    n = qkv.shape[0]
    for nm, t in (("positions", positions), ("cos_sin_cache", cos_sin_cache),
                  ("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _require_cuda(nm, t)
    pos = positions.reshape(-1)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    if pos.shape[0] != n:
        raise ValueError(f"positions must have {n} entries")
    pos = pos.contiguous()
    cache = cos_sin_cache
    if cache.dtype != torch.float32 or cache.dim() != 2 or cache.shape[1] != HEAD_DIM:
        raise ValueError("cos_sin_cache must be fp32 [max_position, 128]")
    cache = cache.contiguous()
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda(name, c)
        _require_dtype(name, c, torch.bfloat16)
        if not c.is_contiguous() or c.shape[-2:] != (num_kv_heads, HEAD_DIM):
            raise ValueError(f"{name} must be a contiguous [..., {num_kv_heads}, 128] bf16 pool")
    sl = slot_mapping.reshape(-1)
    if sl.dtype != torch.int32:
        sl = sl.to(torch.int32)
    if sl.shape[0] != n:
        raise ValueError(f"slot_mapping must have {n} entries")
    sl = sl.contiguous()
    n_slots = k_cache.numel() // (num_kv_heads * HEAD_DIM)
    qw = q_norm_weight.to(torch.bfloat16).contiguous()
    kw = k_norm_weight.to(torch.bfloat16).contiguous()
    q = torch.empty((n, num_q_heads, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    check(lib().qmi_qk_norm_rope_store(
        qkv.data_ptr(), qkv.stride(0), n, num_q_heads, num_kv_heads, HEAD_DIM, qw.data_ptr(),
        kw.data_ptr(), pos.data_ptr(), cache.data_ptr(), cache.shape[0], q.data_ptr(),
        q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), sl.data_ptr(), n_slots, float(eps),
        stream_handle(qkv.device)), "qk_norm_rope_store")
    return q


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` of a fused ``[..., 2 * inter]`` projection (one bf16 rounding)."""
    g2 = _rows2d("gate_up", gate_up)
    inter = g2.shape[1] // 2
    out = torch.empty((g2.shape[0], inter), dtype=torch.bfloat16, device=g2.device)
    check(lib().qmi_silu_mul(g2.data_ptr(), g2.stride(0), g2.shape[0], inter, out.data_ptr(),
                             out.stride(0), stream_handle(g2.device)),
          "silu_mul")
    return out.view(*gate_up.shape[:-1], inter)


# ---------------------------------------------------------------------------
# Decode-batch projections (qwen3_naive.py:427-428, :654, :683, :692-702)
# ---------------------------------------------------------------------------
LINEAR_ROWS_MAX = 256


class RowParts:
    """A projection ``x W^T`` held as fp32 partial products ``parts [S, M, N]``
    (their sum); the residual add + RMSNorm that follows consumes them
    (``add_rms_norm_parts``)."""

    __slots__ = ("parts",)

    def __init__(self, parts: torch.Tensor):
        self.parts = parts

    @property
    def shape(self):
        return self.parts.shape[1:]

    def dense(self) -> torch.Tensor:
        """The projection's bf16 output (one rounding of the fp32 sum)."""
        return self.parts.sum(0).to(torch.bfloat16)


def linear_rows_ok(x: torch.Tensor, weight: torch.Tensor, swiglu: bool = False) -> bool:
    """Whether ``qmi_linear_rows`` takes ``x [M, K] @ weight[N, K]^T``: bf16 GPU
    tensors, 1 <= M <= 256, K % 128 == 0, output width % 16 == 0."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or x.dim() != 2:
        return False
    if not (x.is_cuda and weight.is_cuda) or weight.dim() != 2:
        return False
    n = weight.shape[0] // 2 if swiglu else weight.shape[0]
    return (0 < x.shape[0] <= LINEAR_ROWS_MAX and x.shape[1] == weight.shape[1]
            and x.shape[1] % 128 == 0 and n % 16 == 0 and (not swiglu or weight.shape[0] % 2 == 0))


def _weight16(weight: torch.Tensor) -> torch.Tensor:
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        return weight.contiguous()
    return weight


def linear_rows(x: torch.Tensor, weight: torch.Tensor, swiglu: bool = False) -> torch.Tensor:
    """``x @ weight.T`` in bf16 for decode batches (``F.linear`` without bias);
    ``swiglu=True``: ``weight`` is the packed ``[gate; up]`` gate_up weight and
    the result is ``silu(x @ gate.T) * (x @ up.T)`` with the rounding points of
    the bf16 GEMM followed by ``silu_mul``."""
    if not linear_rows_ok(x, weight, swiglu):
        raise ValueError(f"linear_rows: unsupported x {tuple(x.shape)} / weight "
                         f"{tuple(weight.shape)} (bf16, <= {LINEAR_ROWS_MAX} rows, K % 128)")
    x2 = _rows2d("x", x)
    w = _weight16(weight)
    m, k = x2.shape
    n = w.shape[0] // 2 if swiglu else w.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=x2.device)
    check(lib().qmi_linear_rows(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), m, n, k,
                                1 if swiglu else 0, y.data_ptr(), y.stride(0),
                                stream_handle(x2.device)),
          "linear_rows")
    return y


def linear_rows_parts(x: torch.Tensor, weight: torch.Tensor) -> RowParts:
    """``x @ weight.T`` as fp32 split-K partial products (see ``RowParts``)."""
    if not linear_rows_ok(x, weight):
        raise ValueError(f"linear_rows_parts: unsupported x {tuple(x.shape)} / weight "
                         f"{tuple(weight.shape)}")
    x2 = _rows2d("x", x)
    w = _weight16(weight)
    m, k = x2.shape
    n = w.shape[0]
    L = lib()
    n_parts = L.qmi_linear_rows_parts_count(m, n, k)
    if n_parts <= 0:
        raise ValueError("linear_rows_parts: unsupported shape")
    parts = torch.empty((n_parts, m, n), dtype=torch.float32, device=x2.device)
    check(L.qmi_linear_rows_parts(x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), m, n, k,
                                  parts.data_ptr(), n_parts, stream_handle(x2.device)),
          "linear_rows_parts")
    return RowParts(parts)


def add_rms_norm_parts(x: RowParts, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """``add_rms_norm`` with ``x`` given as partial products: ``s = bf16(sum
    parts) + residual``; returns ``(rms_norm(s), bf16(s))``."""
    parts = x.parts
    r2 = _rows2d("residual", residual)
    if parts.dim() != 3 or tuple(parts.shape[1:]) != tuple(r2.shape) or not parts.is_contiguous():
        raise ValueError("parts must be a contiguous [S, M, N] tensor matching residual [M, N]")
    w = weight.to(torch.bfloat16).contiguous()
    y = torch.empty(r2.shape, dtype=torch.bfloat16, device=r2.device)
    r_out = torch.empty_like(y)
    check(lib().qmi_add_rms_norm_parts(parts.data_ptr(), parts.shape[0], r2.shape[0], r2.data_ptr(),
                                       r2.stride(0), r_out.data_ptr(), r_out.stride(0), w.data_ptr(),
                                       y.data_ptr(), y.stride(0), r2.shape[1], float(eps),
                                       stream_handle(r2.device)),
          "add_rms_norm_parts")
    return y.view(residual.shape), r_out.view(residual.shape)


# ---------------------------------------------------------------------------
# Log-softmax gather (qwen3_grpo_train.py:46-53)
# ---------------------------------------------------------------------------
def _rows_view(logits: torch.Tensor, ids: torch.Tensor):
    """Normalise ``logits`` to [B, T, V] and ``ids`` to [B, T] views."""
    _require_cuda("logits", logits)
    _require_dtype("logits", logits, torch.bfloat16)
    _require_cuda("ids", ids)
    _require_dtype("ids", ids, torch.int64)
    if logits.dim() == 2:
        logits = logits.unsqueeze(0)
    if ids.dim() == 1:
        ids = ids.unsqueeze(0)
    if logits.dim() != 3 or ids.dim() != 2 or tuple(logits.shape[:2]) != tuple(ids.shape):
        raise ValueError(f"logits [B,T,V] / ids [B,T] mismatch: {tuple(logits.shape)} vs "
                         f"{tuple(ids.shape)}")
    if logits.stride(2) != 1:
        logits = logits.contiguous()
    return logits, ids


def logprob_gather(logits: torch.Tensor, ids: torch.Tensor, need_lse: bool = True):
    """``log_softmax(logits.float(), -1).gather(-1, ids[..., None])[..., 0]`` and the row lse.

    ``logits``: ``[B, T, V]`` (or ``[N, V]``) bf16 with unit vocab stride;
    ``ids``: int64 ``[B, T]`` (or ``[N]``).  Returns fp32 ``(lp, lse)`` shaped
    like ``ids``.
    """
    shape = ids.shape
    lg, ii = _rows_view(logits, ids)
    bsz, t, v = lg.shape
    lp = torch.empty((bsz, t), dtype=torch.float32, device=lg.device)
    lse = torch.empty((bsz, t), dtype=torch.float32, device=lg.device) if need_lse else None
    st = lib().qmi_logprob_gather(lg.data_ptr(), lg.stride(0), lg.stride(1), ii.data_ptr(),
                                  ii.stride(0), ii.stride(1), bsz, t, v, lp.data_ptr(),
                                  _ptr(lse), stream_handle(lg.device))
    check(st, "logprob_gather")
    return lp.view(shape), (lse.view(shape) if lse is not None else None)


def sample_tokens(logits: torch.Tensor, temperature: float = 1.0, seed: int | None = None,
                  offset: int = 0, want_logprobs: bool = True):
    """Draw one token per row from ``softmax(logits.float() / temperature)`` and
    return ``(tokens int64 [N], log_softmax(...)[token] fp32 [N] or None)``.

    ``logits``: ``[N, V]`` bf16 with unit vocab stride.  ``seed`` defaults to a
    draw from torch's default CPU generator, so ``torch.manual_seed`` makes
    the tokens reproducible; the same ``(seed, offset)`` gives the same tokens.
    """
    _require_cuda("logits", logits)
    _require_dtype("logits", logits, torch.bfloat16)
    if logits.dim() != 2:
        raise ValueError(f"logits must be [N, V], got {tuple(logits.shape)}")
    if not (temperature > 0.0) or temperature == float("inf"):
        raise ValueError(f"temperature must be finite and > 0, got {temperature}")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    n, v = logits.shape
    if seed is None:
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    tok = torch.empty((n,), dtype=torch.int64, device=logits.device)
    lp = torch.empty((n,), dtype=torch.float32, device=logits.device) if want_logprobs else None
    st = lib().qmi_sample_tokens(logits.data_ptr(), logits.stride(0), n, v, float(temperature),
                                 int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 64 - 1),
                                 tok.data_ptr(), _ptr(lp), stream_handle(logits.device))
    check(st, "sample_tokens")
    return tok, lp


def sample_tokens_topk(logits: torch.Tensor, top_k: int, temperature: float = 1.0,
                       seed: int | None = None, offset: int = 0, want_logprobs: bool = True):
    """Top-k sampling (qwen3_naive.py:1413-1422 / :1641-1650): keep the ``top_k``
    largest of ``logits.float() / temperature`` per row, draw from their softmax
    and return ``(tokens int64 [N], log-probabilities fp32 [N] or None)``.  Of
    entries tied at the k-th value the lowest indices are kept.  ``seed``
    defaults to a draw from torch's default CPU generator."""
    _require_cuda("logits", logits)
    _require_dtype("logits", logits, torch.bfloat16)
    if logits.dim() != 2:
        raise ValueError(f"logits must be [N, V], got {tuple(logits.shape)}")
    n, v = logits.shape
    if not 1 <= int(top_k) <= min(v, 1024):
        raise ValueError(f"top_k must be in [1, min(vocab, 1024)], got {top_k}")
    if not (temperature > 0.0) or temperature == float("inf"):
        raise ValueError(f"temperature must be finite and > 0, got {temperature}")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    if seed is None:
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    tok = torch.empty((n,), dtype=torch.int64, device=logits.device)
    lp = torch.empty((n,), dtype=torch.float32, device=logits.device) if want_logprobs else None
    st = lib().qmi_sample_tokens_topk(logits.data_ptr(), logits.stride(0), n, v, int(top_k),
                                      float(temperature), int(seed) & (2 ** 64 - 1),
                                      int(offset) & (2 ** 64 - 1), tok.data_ptr(), _ptr(lp),
                                      stream_handle(logits.device))
    check(st, "sample_tokens_topk")
    return tok, lp


MAX_FUSED_TOP_K = 64            # largest k the fused lm_head top-k sampler takes
MAX_FUSED_TOP_K_VOCAB = 262144  # and the largest vocabulary it takes it over


def _lm_head_args(hidden: torch.Tensor, weight: torch.Tensor, top_k: int = 0):
    for n, t in (("hidden", hidden), ("weight", weight)):
        _require_cuda(n, t)
        _require_dtype(n, t, torch.bfloat16)
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"hidden [N, H] and weight [V, H] must share H, got {tuple(hidden.shape)} "
                         f"and {tuple(weight.shape)}")
    if hidden.shape[1] % 64 or hidden.shape[1] > 16384:
        raise ValueError(f"hidden size must be a multiple of 64 and at most 16384, got "
                         f"{hidden.shape[1]}")
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        raise ValueError("weight rows must be contiguous, 16-byte aligned, stride % 8 == 0")
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.contiguous()
    n, hdim = hidden.shape
    v = weight.shape[0]
    nbytes = lib().qmi_lm_head_workspace_bytes(n, v, int(top_k))
    ws = torch.empty((max(nbytes, 16) + 15) // 16 * 16, dtype=torch.uint8, device=hidden.device)
    return hidden, n, v, hdim, ws


def lm_head_sample(hidden: torch.Tensor, weight: torch.Tensor, temperature: float = 1.0,
                   seed: int | None = None, offset: int = 0, want_logprobs: bool = True,
                   top_k: int | None = None, row_counters: torch.Tensor | None = None):
    """``logits = bf16(hidden @ weight.T)`` (never materialised), then one token
    per row drawn from ``softmax(logits / temperature)`` -- or, with ``top_k``,
    from the softmax of its ``top_k`` largest entries (ties at the k-th value
    keep the lowest indices) -- and its log-probability under that
    distribution (qwen3_naive.py:1387 / :1607 lm_head, :1413-1423 /
    :1636-1650 sampling).  ``top_k`` up to ``MAX_FUSED_TOP_K``.  Returns
    ``(tokens int64 [N], logprobs fp32 [N] or None)``.

    The draw is inverse transform sampling with one Philox4x32-10 uniform per
    row: counter (0, lo32(q), lo32(offset) + hi32(q), hi32(offset)), key seed,
    where q is ``row_counters[r]`` (int64 ``[N]`` on the device) or the row
    index.  ``seed`` defaults to a draw from torch's default CPU generator, so
    ``torch.manual_seed`` makes the tokens reproducible."""
    if not (temperature > 0.0) or temperature == float("inf"):
        raise ValueError(f"temperature must be finite and > 0, got {temperature}")
    k = 0 if top_k is None else int(top_k)
    if not 0 <= k <= MAX_FUSED_TOP_K:
        raise ValueError(f"top_k must be None or in [1, {MAX_FUSED_TOP_K}], got {top_k}")
    if 0 < k < weight.shape[0] and weight.shape[0] > MAX_FUSED_TOP_K_VOCAB:
        raise ValueError(f"fused top-k takes vocabularies up to {MAX_FUSED_TOP_K_VOCAB}")
    hidden, n, v, hdim, ws = _lm_head_args(hidden, weight, k)
    if seed is None:
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    tok = torch.empty((n,), dtype=torch.int64, device=hidden.device)
    lp = torch.empty((n,), dtype=torch.float32, device=hidden.device) if want_logprobs else None
    if n == 0:
        return tok, lp
    rc = None
    if row_counters is not None:
        _require_cuda("row_counters", row_counters)
        _require_dtype("row_counters", row_counters, torch.int64)
        if row_counters.shape != (n,):
            raise ValueError(f"row_counters must be [{n}], got {tuple(row_counters.shape)}")
        rc = row_counters.contiguous()
    st = lib().qmi_lm_head_sample(hidden.data_ptr(), hidden.stride(0), n, weight.data_ptr(),
                                  weight.stride(0), v, hdim, float(temperature), k,
                                  int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 64 - 1),
                                  _ptr(rc), tok.data_ptr(), _ptr(lp), ws.data_ptr(), ws.numel(),
                                  stream_handle(hidden.device))
    check(st, "lm_head_sample")
    return tok, lp


def lm_head_logprob(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor):
    """``log_softmax(bf16(hidden @ weight.T))[targets]`` per row without
    materialising the logits (lm_head + qwen3_grpo_train.py:46-53's gather).
    ``targets``: int64 ``[N]``; a target outside the vocabulary gives NaN.
    Returns ``(logprobs fp32 [N], lse fp32 [N])``."""
    hidden, n, v, hdim, ws = _lm_head_args(hidden, weight)
    _require_cuda("targets", targets)
    tg = targets.reshape(-1).to(torch.int64)
    if tg.shape[0] != n:
        raise ValueError(f"targets must have {n} entries, got {tg.shape[0]}")
    lp = torch.empty((n,), dtype=torch.float32, device=hidden.device)
    lse = torch.empty_like(lp)
    if n == 0:
        return lp, lse
    st = lib().qmi_lm_head_logprob(hidden.data_ptr(), hidden.stride(0), n, weight.data_ptr(),
                                   weight.stride(0), v, hdim, tg.data_ptr(), tg.stride(0),
                                   lp.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(),
                                   stream_handle(hidden.device))
    check(st, "lm_head_logprob")
    return lp, lse


def logprob_gather_backward(logits: torch.Tensor, ids: torch.Tensor, lse: torch.Tensor,
                            coef: torch.Tensor, grad_scale: torch.Tensor | None = None,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """``grad[b,t,v] = g * coef[b,t] * (1[v==id] - exp(logits[b,t,v] - lse[b,t]))`` in bf16."""
    lshape = logits.shape
    lg, ii = _rows_view(logits, ids)
    bsz, t, v = lg.shape
    coef = coef.reshape(bsz, t).float().contiguous()
    lse = lse.reshape(bsz, t).float().contiguous()
    if grad_scale is not None:
        grad_scale = grad_scale.reshape(1).float().contiguous()
    if out is None:
        out = torch.empty((bsz, t, v), dtype=torch.bfloat16, device=lg.device)
    else:
        out = out.view(bsz, t, v)
        if out.stride(2) != 1:
            raise ValueError("grad out must have unit vocab stride")
    st = lib().qmi_logprob_gather_backward(
        lg.data_ptr(), lg.stride(0), lg.stride(1), ii.data_ptr(), ii.stride(0), ii.stride(1),
        bsz, t, v, lse.data_ptr(), coef.data_ptr(), _ptr(grad_scale), out.data_ptr(),
        out.stride(0), out.stride(1), stream_handle(lg.device))
    check(st, "logprob_gather_backward")
    return out.view(lshape)


# ---------------------------------------------------------------------------
# Advantages / clipped loss (qwen3_grpo_train.py:162-199)
# ---------------------------------------------------------------------------
def grpo_advantage(rewards: torch.Tensor, prompt_ids: torch.Tensor, eps: float = 1e-8):
    """Group-normalised advantages ``(r - mean_g) / (std_g + eps)`` (unbiased std)."""
    _require_cuda("rewards", rewards)
    _require_cuda("prompt_ids", prompt_ids)
    r = rewards.reshape(-1).float().contiguous()
    p = prompt_ids.reshape(-1).to(torch.int64).contiguous()
    if r.shape != p.shape:
        raise ValueError("rewards and prompt_ids must have the same length")
    out = torch.empty_like(r)
    if r.numel():
        check(lib().qmi_grpo_advantage(r.data_ptr(), p.data_ptr(), r.numel(), float(eps),
                                       out.data_ptr(), stream_handle(r.device)),
              "grpo_advantage")
    return out


def ppo_clipped_loss_fwd(new_lp: torch.Tensor, old_lp: torch.Tensor, adv: torch.Tensor,
                         mask: torch.Tensor, clip_eps: float = 0.2, reduction: str = "token",
                         need_grad: bool = True):
    """Clipped surrogate on ``[B, T]`` log-probs; ``adv`` is ``[B, T]`` or ``[B]``.

    Returns ``(loss, dloss_dnew)`` (fp32 scalar tensor, fp32 ``[B, T]`` or None).
    """
    for n, t in (("new_lp", new_lp), ("old_lp", old_lp), ("mask", mask), ("adv", adv)):
        _require_cuda(n, t)
    if new_lp.dim() == 1:
        new_lp, old_lp, mask = new_lp[None], old_lp[None], mask[None]
        adv = adv[None] if adv.dim() == 1 and adv.shape[0] == new_lp.shape[1] else adv
    bsz, t = new_lp.shape
    nw = new_lp.float().contiguous()
    od = old_lp.float().reshape(bsz, t).contiguous()
    mk = mask.float().reshape(bsz, t).contiguous()
    av = adv.float()
    if av.dim() == 1 and av.shape[0] == bsz:
        av = av.contiguous()
        ass, ats = 1, 0
    else:
        av = av.reshape(bsz, t).contiguous()
        ass, ats = t, 1
    loss = torch.empty((), dtype=torch.float32, device=nw.device)
    dlp = torch.empty((bsz, t), dtype=torch.float32, device=nw.device) if need_grad else None
    check(lib().qmi_ppo_clipped_loss(nw.data_ptr(), od.data_ptr(), mk.data_ptr(), av.data_ptr(),
                                     ass, ats, bsz, t, float(clip_eps), REDUCTIONS[reduction],
                                     loss.data_ptr(), _ptr(dlp), stream_handle(nw.device)),
          "ppo_clipped_loss")
    return loss, dlp


def grpo_fused_forward(logits: torch.Tensor, ids: torch.Tensor, old_lp: torch.Tensor,
                       mask: torch.Tensor, rewards: torch.Tensor, prompt_ids: torch.Tensor,
                       adv_eps: float = 1e-8, clip_eps: float = 0.2, reduction: str = "token"):
    """One streaming pass: per-token logprob + lse, group advantages, loss, d loss / d lp.

    ``logits [B, T, V]`` bf16 rows are aligned with ``ids [B, T]`` (pass
    ``logits[:, :-1]`` / ``ids[:, 1:]`` for next-token alignment).
    Returns a dict of fp32 tensors: loss (scalar), lp, lse, dlp ``[B, T]``, adv ``[B]``.
    """
    lg, ii = _rows_view(logits, ids)
    bsz, t, v = lg.shape
    dev = lg.device
    od = old_lp.float().reshape(bsz, t).contiguous()
    mk = mask.float().reshape(bsz, t).contiguous()
    rw = rewards.float().reshape(bsz).contiguous()
    pid = prompt_ids.to(torch.int64).reshape(bsz).contiguous()
    lp = torch.empty((bsz, t), dtype=torch.float32, device=dev)
    lse = torch.empty_like(lp)
    dlp = torch.empty_like(lp)
    adv = torch.empty((bsz,), dtype=torch.float32, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    L = lib()
    nbytes = L.qmi_grpo_fused_workspace_bytes(bsz, t)
    # Per-sequence sums only; the kernels keep no state in it between calls.
    ws = torch.empty(((nbytes + 15) // 16) * 16, dtype=torch.uint8, device=dev)
    check(L.qmi_grpo_fused_loss(lg.data_ptr(), lg.stride(0), lg.stride(1), ii.data_ptr(),
                                ii.stride(0), ii.stride(1), bsz, t, v, od.data_ptr(),
                                mk.data_ptr(), rw.data_ptr(), pid.data_ptr(), float(adv_eps),
                                float(clip_eps), REDUCTIONS[reduction], lp.data_ptr(),
                                lse.data_ptr(), adv.data_ptr(), dlp.data_ptr(), loss.data_ptr(),
                                ws.data_ptr(), ws.numel(), stream_handle(dev)),
          "grpo_fused_loss")
    return {"loss": loss, "lp": lp, "lse": lse, "dlp": dlp, "adv": adv}


def library_version() -> int:
    return lib().qmi_version()
