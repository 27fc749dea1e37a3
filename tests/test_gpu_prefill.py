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


def test_prefill_config4_step(pkg, gpu):
    """First chunk step of the prefix-cache workload: 16 sequences, 512 cached
    prefix tokens in 2 shared pages, 512-token chunks (8,192 query rows)."""
    sched = W.prefix_prefill_chunks(seed=0)
    step = sched["steps"][0]
    n_blocks = 2 + 16 * 16
    inp = W.prefill_step_inputs(0, step, [0, 1], n_blocks)
    g = torch.Generator().manual_seed(15)
    kc = torch.randn(n_blocks, 256, 8, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, 256, 8, 128, generator=g).to(torch.bfloat16)
    print("[prefill] config4 step", flush=True)
    cu_q = inp["cu_seqlens_q"].tolist()
    cu_k = inp["cu_seqlens_k"].tolist()
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
