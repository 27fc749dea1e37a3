"""Varlen paged causal prefill parity against the oracle (tolerance: max abs
2e-2 in bf16, as for the reference path)."""
import pytest
import torch

from oracle import attention as OA
from oracle import workloads as W

pytestmark = pytest.mark.gpu

TOL = 2e-2
SCALE = 128 ** -0.5


def _pool(seed, lens_k, hkv=8, extra=2):
    """Random paged pool and shuffled block tables for sequences of lens_k keys."""
    g = torch.Generator().manual_seed(seed)
    need = [max(1, (L + 255) // 256) for L in lens_k]
    nb = sum(need) + extra
    perm = torch.randperm(nb, generator=g)
    width = max(need)
    bt = torch.full((len(lens_k), width), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kc = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16)
    return kc, vc, bt


def _run(pkg, gpu, q, kc, vc, cu_q, cu_k, bt):
    cq = torch.tensor(cu_q, dtype=torch.int32)
    ck = torch.tensor(cu_k, dtype=torch.int32)
    max_q = max(cu_q[i + 1] - cu_q[i] for i in range(len(cu_q) - 1))
    max_k = max(cu_k[i + 1] - cu_k[i] for i in range(len(cu_k) - 1))
    out = pkg.kernels.varlen_prefill_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), cq.to(gpu),
                                               ck.to(gpu), max_q, max_k, SCALE, True, bt.to(gpu))
    torch.cuda.synchronize()
    return out


def _check(out, q, kc, vc, cu_q, cu_k, bt, tol=TOL):
    ref = OA.varlen_prefill(q, kc, vc, cu_q, cu_k, bt, SCALE)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= tol, f"max abs err {err}"
    return err


@pytest.mark.parametrize("L", [1, 15, 16, 17, 63, 64, 65, 255, 256, 257, 700])
def test_prefill_full_causal_lengths(pkg, gpu, L):
    kc, vc, bt = _pool(L, [L])
    g = torch.Generator().manual_seed(100 + L)
    q = torch.randn(L, 16, 128, generator=g).to(torch.bfloat16)
    print(f"[prefill] full causal L={L}", flush=True)
    out = _run(pkg, gpu, q, kc, vc, [0, L], [0, L], bt)
    _check(out, q, kc, vc, [0, L], [0, L], bt)


@pytest.mark.parametrize("prefix,chunk", [(512, 512), (256, 37), (700, 1), (1, 300), (300, 300)])
def test_prefill_prefix_cached_chunk(pkg, gpu, prefix, chunk):
    """New tokens see the whole cached prefix (bottom-right causal alignment)."""
    Lk = prefix + chunk
    kc, vc, bt = _pool(prefix * 7 + chunk, [Lk])
    g = torch.Generator().manual_seed(prefix + chunk)
    q = torch.randn(chunk, 16, 128, generator=g).to(torch.bfloat16)
    print(f"[prefill] prefix={prefix} chunk={chunk}", flush=True)
    out = _run(pkg, gpu, q, kc, vc, [0, chunk], [0, Lk], bt)
    _check(out, q, kc, vc, [0, chunk], [0, Lk], bt)


def test_prefill_mixed_batch_decode_and_chunks(pkg, gpu):
    """Mixed step as in the reference's mixed-batch case: two decode rows and a
    512-token chunk, plus an empty sequence and a short prefill."""
    lens_q = [1, 1, 512, 0, 40]
    lens_k = [41, 13, 512, 5, 40]
    cu_q, cu_k = [0], [0]
    for a, c in zip(lens_q, lens_k):
        cu_q.append(cu_q[-1] + a)
        cu_k.append(cu_k[-1] + c)
    kc, vc, bt = _pool(7, lens_k)
    g = torch.Generator().manual_seed(8)
    q = torch.randn(cu_q[-1], 16, 128, generator=g).to(torch.bfloat16)
    print("[prefill] mixed batch", flush=True)
    out = _run(pkg, gpu, q, kc, vc, cu_q, cu_k, bt)
    _check(out, q, kc, vc, cu_q, cu_k, bt)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (16, 4)])
def test_prefill_gqa_ratios(pkg, gpu, hq, hkv):
    lens_q, lens_k = [100, 333], [356, 333]
    cu_q = [0, 100, 433]
    cu_k = [0, 356, 689]
    kc, vc, bt = _pool(9 + hq, lens_k, hkv=hkv)
    g = torch.Generator().manual_seed(10 + hq + hkv)
    q = torch.randn(433, hq, 128, generator=g).to(torch.bfloat16)
    print(f"[prefill] gqa {hq}/{hkv}", flush=True)
    out = _run(pkg, gpu, q, kc, vc, cu_q, cu_k, bt)
    _check(out, q, kc, vc, cu_q, cu_k, bt)


def test_prefill_strided_q_view(pkg, gpu):
    g = torch.Generator().manual_seed(11)
    L = 130
    qkv = torch.randn(L, 4096, generator=g).to(torch.bfloat16)
    q = qkv[:, :2048].view(L, 16, 128)
    kc, vc, bt = _pool(12, [L])
    print("[prefill] strided q", flush=True)
    cq = torch.tensor([0, L], dtype=torch.int32, device=gpu)
    out = pkg.kernels.varlen_prefill_attention(qkv.to(gpu)[:, :2048].view(L, 16, 128), kc.to(gpu),
                                               vc.to(gpu), cq, cq, L, L, SCALE, True, bt.to(gpu))
    torch.cuda.synchronize()
    _check(out, q, kc, vc, [0, L], [0, L], bt)


def test_prefill_chunked_equals_unchunked(pkg, gpu):
    """The exact-math form of the reference's chunked-vs-unchunked check
    (test_chunked_prefill.py:63-155): a 1100-token prompt processed whole and
    in 256-token chunks over the same cache gives the same outputs."""
    L = 1100
    kc, vc, bt = _pool(13, [L])
    g = torch.Generator().manual_seed(14)
    q = torch.randn(L, 16, 128, generator=g).to(torch.bfloat16)
    print("[prefill] chunked == unchunked", flush=True)
    full = _run(pkg, gpu, q, kc, vc, [0, L], [0, L], bt)
    parts = []
    for s in range(0, L, 256):
        e = min(L, s + 256)
        parts.append(_run(pkg, gpu, q[s:e], kc, vc, [0, e - s], [0, e], bt))
    chunked = torch.cat(parts)
    assert (chunked.float() - full.float()).abs().max().item() <= 1e-2
    _check(full, q, kc, vc, [0, L], [0, L], bt)


_CONFIG4 = W.prefix_prefill_chunks(seed=0)


@pytest.mark.parametrize("step_idx", range(len(_CONFIG4["steps"])))
def test_prefill_config4_step(pkg, gpu, step_idx):
    """Every chunk step of the prefix-cache workload: 16 sequences, 512 cached
    prefix tokens in 2 shared pages, 512-token chunks.  Step 1 has 8,192 query
    rows; the later steps carry the longest key ranges (up to 2,560 keys),
    fewer sequences and the launch tails.  Every sequence of the step is
    compared with the oracle."""
    step = _CONFIG4["steps"][step_idx]
    n_blocks = 2 + 16 * 16
    inp = W.prefill_step_inputs(0, step, [0, 1], n_blocks)
    g = torch.Generator().manual_seed(15)
    kc = torch.randn(n_blocks, 256, 8, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, 256, 8, 128, generator=g).to(torch.bfloat16)
    cu_q = inp["cu_seqlens_q"].tolist()
    cu_k = inp["cu_seqlens_k"].tolist()
    print(f"[prefill] config4 step {step_idx + 1}/{len(_CONFIG4['steps'])}: {len(step)} seqs, "
          f"{cu_q[-1]} queries, max keys {inp['max_seqlen_k']}", flush=True)
    out = _run(pkg, gpu, inp["q"], kc, vc, cu_q, cu_k, inp["block_tables"])
    _check(out, inp["q"], kc, vc, cu_q, cu_k, inp["block_tables"])


def test_prefill_graph_replay_matches_eager(pkg, gpu):
    kc, vc, bt = _pool(16, [300, 90])
    g = torch.Generator().manual_seed(17)
    q = torch.randn(150, 16, 128, generator=g).to(torch.bfloat16).to(gpu)
    cq = torch.tensor([0, 100, 150], dtype=torch.int32, device=gpu)
    ck = torch.tensor([0, 300, 390], dtype=torch.int32, device=gpu)
    kcg, vcg, btg = kc.to(gpu), vc.to(gpu), bt.to(gpu)
    print("[prefill] graph capture", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.kernels.varlen_prefill_attention(q, kcg, vcg, cq, ck, 100, 300, SCALE, True, btg)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.kernels.varlen_prefill_attention(q, kcg, vcg, cq, ck, 100, 300, SCALE, True, btg)
    for it in range(3):
        q.copy_(torch.randn(q.shape, generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        eager = pkg.kernels.varlen_prefill_attention(q, kcg, vcg, cq, ck, 100, 300, SCALE, True, btg)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def _queue_case(gpu, n_seqs, seed):
    """A launch on the persistent work queue (its counters live in the
    workspace): n_seqs 512-token chunks after a 1,024-token prefix."""
    lens_q = [512] * n_seqs
    lens_k = [1024 + n for n in lens_q]
    kc, vc, bt = _pool(seed, lens_k)
    cu_q, cu_k = [0], [0]
    for a, c in zip(lens_q, lens_k):
        cu_q.append(cu_q[-1] + a)
        cu_k.append(cu_k[-1] + c)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(cu_q[-1], 16, 128, generator=g).to(torch.bfloat16)
    args = (q.to(gpu), kc.to(gpu), vc.to(gpu), torch.tensor(cu_q, dtype=torch.int32, device=gpu),
            torch.tensor(cu_k, dtype=torch.int32, device=gpu), 512, max(lens_k), SCALE, True,
            bt.to(gpu))
    return args, (q, kc, vc, cu_q, cu_k, bt)


def test_prefill_graph_keeps_private_workspace(pkg, gpu):
    """A captured prefill owns its workspace: an eager call that outgrows the
    cached workspace (which frees it) before the replays changes nothing, and
    every replay equals the eager result."""
    small, ref_small = _queue_case(gpu, 10, 60)
    big, _ = _queue_case(gpu, 20, 61)
    print("[prefill] graph with private workspace", flush=True)
    eager0 = pkg.kernels.varlen_prefill_attention(*small)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.kernels.varlen_prefill_attention(*small)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.kernels.varlen_prefill_attention(*small)
    for it in range(3):
        pkg.kernels.varlen_prefill_attention(*big)     # grows (replaces) the cached workspace
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager0), it
        assert torch.equal(pkg.kernels.varlen_prefill_attention(*small), eager0)
    _check(out, *ref_small)


def test_prefill_two_streams_do_not_share_counters(pkg, gpu):
    """Prefill calls on two streams at once (each stream its own cached
    workspace, so the work-queue counters are never shared) give the results
    of the calls made one after the other."""
    a, _ = _queue_case(gpu, 10, 70)
    b, _ = _queue_case(gpu, 12, 71)
    want_a = pkg.kernels.varlen_prefill_attention(*a).clone()
    want_b = pkg.kernels.varlen_prefill_attention(*b).clone()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    print("[prefill] two streams", flush=True)
    for it in range(3):
        s1.wait_stream(torch.cuda.current_stream())
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s1):
            out_a = pkg.kernels.varlen_prefill_attention(*a)
        with torch.cuda.stream(s2):
            out_b = pkg.kernels.varlen_prefill_attention(*b)
        torch.cuda.synchronize()
        assert torch.equal(out_a, want_a) and torch.equal(out_b, want_b), it


def test_prefill_rejects_bad_inputs(pkg, gpu):
    kc, vc, bt = _pool(18, [10])
    q = torch.zeros(10, 16, 128, dtype=torch.bfloat16, device=gpu)
    cq = torch.tensor([0, 10], dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        pkg.kernels.varlen_prefill_attention(q, kc.to(gpu), vc.to(gpu), cq, cq, 10, 10, SCALE,
                                             False, bt.to(gpu))
    with pytest.raises(ValueError):
        pkg.kernels.varlen_prefill_attention(q, kc.to(gpu), vc.to(gpu), cq, cq, 10, 10, SCALE,
                                             True, None)


def test_prefill_unmapped_page_contributes_nothing(pkg, gpu):
    """Keys on a page whose table entry is -1 are ignored, as in decode: 8
    queries at the end of a 300-key sequence whose second page is unmapped
    attend exactly to the 256 keys of the first page (each query's causal
    horizon is past key 255), which is decode attention over that page."""
    kc, vc, bt = _pool(90, [300])
    bt[0, 1] = -1
    g = torch.Generator().manual_seed(91)
    q = torch.randn(8, 16, 128, generator=g).to(torch.bfloat16)
    print("[prefill] unmapped page", flush=True)
    out = _run(pkg, gpu, q, kc, vc, [0, 8], [0, 300], bt)
    ref = OA.paged_decode(q, kc, vc, torch.full((8,), 256, dtype=torch.int32),
                          bt[:, :1].repeat(8, 1), SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


def test_prefill_rejects_empty_pool(pkg, gpu):
    kc = torch.zeros(0, 256, 8, 128, dtype=torch.bfloat16, device=gpu)
    q = torch.zeros(4, 16, 128, dtype=torch.bfloat16, device=gpu)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=gpu)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=gpu)
    with pytest.raises((ValueError, RuntimeError)):
        pkg.kernels.varlen_prefill_attention(q, kc, kc, cu, cu, 4, 4, SCALE, True, bt)


def _run_split(pkg, gpu, q, kc, vc, cu_q, cu_k, bt, split_keys, max_k=None):
    cq = torch.tensor(cu_q, dtype=torch.int32)
    ck = torch.tensor(cu_k, dtype=torch.int32)
    max_q = max(cu_q[i + 1] - cu_q[i] for i in range(len(cu_q) - 1))
    if max_k is None:
        max_k = max(cu_k[i + 1] - cu_k[i] for i in range(len(cu_k) - 1))
    out = pkg.kernels.varlen_prefill_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), cq.to(gpu),
                                               ck.to(gpu), max_q, max_k, SCALE, True, bt.to(gpu),
                                               split_keys=split_keys)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("split_keys", [64, 128, 320, 1024])
@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4)])
def test_prefill_split_key_ranges(pkg, gpu, split_keys, hq, hkv):
    """Key ranges split across workgroups and merged give the oracle's result:
    decode-like rows, a prefix-cached chunk, a full causal prompt, an empty
    sequence and a short one, with pieces from one tile up."""
    lens_q = [1, 200, 1300, 0, 37]
    lens_k = [1500, 900, 1300, 3, 37]
    cu_q, cu_k = [0], [0]
    for a, c in zip(lens_q, lens_k):
        cu_q.append(cu_q[-1] + a)
        cu_k.append(cu_k[-1] + c)
    kc, vc, bt = _pool(40 + split_keys + hq, lens_k, hkv=hkv)
    g = torch.Generator().manual_seed(41 + split_keys)
    q = torch.randn(cu_q[-1], hq, 128, generator=g).to(torch.bfloat16)
    print(f"[prefill] split_keys={split_keys} gqa {hq}/{hkv}", flush=True)
    n_ws = pkg._lib.lib().qmi_varlen_prefill_workspace_bytes(5, 1300, 1500, hq, hkv, bt.shape[1],
                                                             split_keys)
    assert n_ws > 0  # the launch is split
    out = _run_split(pkg, gpu, q, kc, vc, cu_q, cu_k, bt, split_keys)
    _check(out, q, kc, vc, cu_q, cu_k, bt)
    whole = _run_split(pkg, gpu, q, kc, vc, cu_q, cu_k, bt, 1 << 20)
    assert (out.float() - whole.float()).abs().max().item() <= 1e-2


def test_prefill_split_any_max_seqlen_k(pkg, gpu):
    """max_seqlen_k only sizes the split: too small (no split) and far too
    large (more pieces than tiles for short rows) both give the oracle's result."""
    lens_k = [1100, 700]
    cu_q, cu_k = [0, 300, 400], [0, 1100, 1800]
    kc, vc, bt = _pool(50, lens_k)
    g = torch.Generator().manual_seed(51)
    q = torch.randn(400, 16, 128, generator=g).to(torch.bfloat16)
    print("[prefill] split with any max_seqlen_k", flush=True)
    ref = OA.varlen_prefill(q, kc, vc, cu_q, cu_k, bt, SCALE)
    for max_k in (1, 1100, 50_000):
        out = _run_split(pkg, gpu, q, kc, vc, cu_q, cu_k, bt, 128, max_k=max_k)
        assert (out.float().cpu() - ref).abs().max().item() <= TOL, max_k


def test_prefill_split_unmapped_page(pkg, gpu):
    """Keys on an unmapped page (table entry -1) inside a split key range
    contribute nothing: 300 queries at the end of a 1100-key sequence whose
    third page (keys 512..767) is unmapped match fp32 attention over the other
    keys under the same causal mask."""
    L, Lq = 1100, 300
    kc, vc, bt = _pool(52, [L])
    bt[0, 2] = -1
    g = torch.Generator().manual_seed(53)
    q = torch.randn(Lq, 16, 128, generator=g).to(torch.bfloat16)
    print("[prefill] split over an unmapped page", flush=True)
    out = _run_split(pkg, gpu, q, kc, vc, [0, Lq], [0, L], bt, 128)
    keys = torch.arange(L)
    pages = bt[0, keys // 256].long()
    mapped = pages >= 0
    rows = pages.clamp(min=0) * 256 + keys % 256
    k = kc.reshape(-1, 8, 128)[rows].float()  # [L, 8, 128]
    v = vc.reshape(-1, 8, 128)[rows].float()
    qi = torch.arange(Lq)[:, None] + (L - Lq)
    visible = (keys[None, :] <= qi) & mapped[None, :]
    ref = torch.empty(Lq, 16, 128)
    for h in range(16):
        sc = (q[:, h].float() @ k[:, h // 2].T) * SCALE
        sc = sc.masked_fill(~visible, float("-inf"))
        ref[:, h] = torch.softmax(sc, dim=-1) @ v[:, h // 2]
    assert (out.float().cpu() - ref).abs().max().item() <= TOL
    whole = _run_split(pkg, gpu, q, kc, vc, [0, Lq], [0, L], bt, 1 << 20)
    assert (out.float() - whole.float()).abs().max().item() <= 1e-2


def test_prefill_split_needs_workspace(pkg, gpu):
    """Through the C ABI: without a workspace the launch runs unsplit and
    gives exactly the unsplit result."""
    import ctypes
    L = 900
    kc, vc, bt = _pool(60, [L])
    g = torch.Generator().manual_seed(61)
    q = torch.randn(L, 16, 128, generator=g).to(torch.bfloat16).to(gpu)
    kcg, vcg, btg = kc.to(gpu), vc.to(gpu), bt.to(gpu)
    cu = torch.tensor([0, L], dtype=torch.int32, device=gpu)
    print("[prefill] split without workspace", flush=True)
    whole = pkg.kernels.varlen_prefill_attention(q, kcg, vcg, cu, cu, L, L, SCALE, True, btg,
                                                 split_keys=1 << 20)
    out = torch.empty_like(whole)
    lib = pkg._lib.lib()
    st = lib.qmi_varlen_prefill_attention(
        q.data_ptr(), q.stride(0), q.stride(1), kcg.data_ptr(), vcg.data_ptr(), kcg.shape[0], 256,
        16, 8, 128, cu.data_ptr(), cu.data_ptr(), btg.data_ptr(), btg.stride(0), btg.shape[1], 1,
        L, L, L, SCALE, out.data_ptr(), out.stride(0), out.stride(1), None, 0, 64,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert st == 0
    assert torch.equal(out, whole)
    with pytest.raises(ValueError):
        pkg.kernels.varlen_prefill_attention(q, kcg, vcg, cu, cu, L, L, SCALE, True, btg,
                                             split_keys=100)


@pytest.mark.parametrize("lq,prefix,hq,hkv", [(1, 4095, 16, 8), (64, 4000, 16, 8), (200, 3000, 16, 4),
                                               (300, 2000, 8, 8)])
def test_prefill_auto_split_long_prefix(pkg, gpu, lq, prefix, hq, hkv):
    """A lone short chunk after a long cached prefix has a handful of work
    items, so the automatic mode splits its key range; the result matches the
    oracle and the unsplit launch."""
    L = prefix + lq
    kc, vc, bt = _pool(70 + lq, [L], hkv=hkv)
    g = torch.Generator().manual_seed(71 + lq)
    q = torch.randn(lq, hq, 128, generator=g).to(torch.bfloat16)
    print(f"[prefill] auto split lq={lq} prefix={prefix} gqa {hq}/{hkv}", flush=True)
    assert pkg._lib.lib().qmi_varlen_prefill_workspace_bytes(1, lq, L, hq, hkv, bt.shape[1], 0) > 0
    out = _run_split(pkg, gpu, q, kc, vc, [0, lq], [0, L], bt, 0)
    _check(out, q, kc, vc, [0, lq], [0, L], bt)
    whole = _run_split(pkg, gpu, q, kc, vc, [0, lq], [0, L], bt, 1 << 20)
    assert (out.float() - whole.float()).abs().max().item() <= 1e-2


def test_prefill_misaligned_q_view(pkg, gpu):
    """q starting mid-allocation (not 16-byte aligned) is copied by the shim."""
    L = 200
    kc, vc, bt = _pool(80, [L])
    g = torch.Generator().manual_seed(81)
    q = torch.randn(L, 16, 128, generator=g).to(torch.bfloat16)
    big = torch.zeros(q.numel() + 8, dtype=torch.bfloat16, device=gpu)
    big[1:1 + q.numel()].copy_(q.reshape(-1).to(gpu))
    qm = big[1:1 + q.numel()].view(q.shape)
    cq = torch.tensor([0, L], dtype=torch.int32, device=gpu)
    print("[prefill] misaligned q", flush=True)
    out = pkg.kernels.varlen_prefill_attention(qm, kc.to(gpu), vc.to(gpu), cq, cq, L, L, SCALE,
                                               True, bt.to(gpu))
    torch.cuda.synchronize()
    _check(out, q, kc, vc, [0, L], [0, L], bt)


@pytest.mark.parametrize("lens_q,prefix,hq,hkv", [
    ([512] * 10, 1024, 16, 8),   # 80 items per KV head: work queue, no split
    ([512] * 4, 2000, 16, 8),    # 32 items per KV head: thin, long items split
    ([1024] * 2, 1500, 16, 4),   # GQA 4: 64 items per KV head, thin
    ([512, 300, 512, 77, 512, 512, 200, 512], 1200, 8, 8),  # GQA 1, ragged chunks, thin
])
def test_prefill_queue_modes(pkg, gpu, lens_q, prefix, hq, hkv):
    """Launches of a few rounds of items run on the persistent work queue
    (thin ones with split items and the merge kernel): they match the oracle,
    two calls on one zeroed workspace give identical results, and the
    queue's counters are back at zero after each call."""
    lens_k = [prefix + n for n in lens_q]
    kc, vc, bt = _pool(90 + len(lens_q) + hq, lens_k, hkv=hkv)
    cu_q, cu_k = [0], [0]
    for a, c in zip(lens_q, lens_k):
        cu_q.append(cu_q[-1] + a)
        cu_k.append(cu_k[-1] + c)
    g = torch.Generator().manual_seed(91 + hq)
    q = torch.randn(cu_q[-1], hq, 128, generator=g).to(torch.bfloat16)
    nbytes = pkg._lib.lib().qmi_varlen_prefill_workspace_bytes(len(lens_q), max(lens_q), max(lens_k),
                                                               hq, hkv, bt.shape[1], 0)
    ws = torch.zeros(nbytes // 4 + 1, dtype=torch.float32, device=gpu)
    args = (q.to(gpu), kc.to(gpu), vc.to(gpu), torch.tensor(cu_q, dtype=torch.int32, device=gpu),
            torch.tensor(cu_k, dtype=torch.int32, device=gpu), max(lens_q), max(lens_k), SCALE,
            True, bt.to(gpu))
    print(f"[prefill] queue mode {len(lens_q)} seqs prefix {prefix} gqa {hq}/{hkv}", flush=True)
    out1 = pkg.kernels.varlen_prefill_attention(*args, workspace=ws)
    torch.cuda.synchronize()
    counters = ws[:hkv + 1].view(torch.int32).cpu()
    assert int(counters.abs().sum()) == 0, counters
    out2 = pkg.kernels.varlen_prefill_attention(*args, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert int(ws[:hkv + 1].view(torch.int32).abs().sum().item()) == 0
    _check(out1, q, kc, vc, cu_q, cu_k, bt)
    # Without the workspace (C ABI, NULL): one workgroup per item, unsplit.
    import ctypes
    whole = torch.empty_like(out1)
    qg, kcg, vcg, cqg, ckg, _, _, _, _, btg = args
    st = pkg._lib.lib().qmi_varlen_prefill_attention(
        qg.data_ptr(), qg.stride(0), qg.stride(1), kcg.data_ptr(), vcg.data_ptr(), kcg.shape[0], 256,
        hq, hkv, 128, cqg.data_ptr(), ckg.data_ptr(), btg.data_ptr(), btg.stride(0), btg.shape[1],
        len(lens_q), max(lens_q), max(lens_k), cu_q[-1], SCALE, whole.data_ptr(), whole.stride(0),
        whole.stride(1), None, 0, 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert st == 0
    assert (out1.float() - whole.float()).abs().max().item() <= 1e-2


@pytest.mark.parametrize("layout", ["head_stride_136", "offset_8_bytes"])
def test_prefill_strided_out_view(pkg, gpu, layout):
    """O written into a view of a larger buffer: rows staged in LDS are stored
    as 8-byte halves when the heads are not contiguous or the view is not
    16-byte aligned; nothing outside the view is touched."""
    lens_q, prefix = [300, 64, 200], 300
    lens_k = [prefix + n for n in lens_q]
    kc, vc, bt = _pool(91, lens_k)
    tq = sum(lens_q)
    g = torch.Generator().manual_seed(92)
    q = torch.randn(tq, 16, 128, generator=g).to(torch.bfloat16)
    cu_q = [0]
    for n in lens_q:
        cu_q.append(cu_q[-1] + n)
    cu_k = [0]
    for n in lens_k:
        cu_k.append(cu_k[-1] + n)
    if layout == "head_stride_136":
        big = torch.zeros(tq, 16, 136, dtype=torch.bfloat16, device=gpu)
        out = big[:, :, 4:132]
    else:
        big = torch.zeros(tq * 16 * 128 + 8, dtype=torch.bfloat16, device=gpu)
        out = big[4:4 + tq * 16 * 128].view(tq, 16, 128)
    print(f"[prefill] strided out {layout}", flush=True)
    res = pkg.kernels.varlen_prefill_attention(
        q.to(gpu), kc.to(gpu), vc.to(gpu), torch.tensor(cu_q, dtype=torch.int32, device=gpu),
        torch.tensor(cu_k, dtype=torch.int32, device=gpu), max(lens_q), max(lens_k), SCALE, True,
        bt.to(gpu), out)
    torch.cuda.synchronize()
    assert res.data_ptr() == out.data_ptr()
    _check(out, q, kc, vc, cu_q, cu_k, bt)
    if layout == "head_stride_136":
        assert not big[:, :, :4].any() and not big[:, :, 132:].any()
    else:
        assert not big[:4].any() and not big[4 + tq * 16 * 128:].any()
