"""Paged decode attention parity against the oracle (tolerance: max abs 2e-2 in
bf16, the bound the reference path is held to)."""
import pytest
import torch

from oracle import attention as OA
from oracle import paged as OP
from oracle import workloads as W

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _decode(pkg, gpu, w, **kw):
    return pkg.kernels.paged_decode_attention(
        w["q"].to(gpu), w["k_cache"].to(gpu), w["v_cache"].to(gpu), w["cache_seqlens"].to(gpu),
        w["block_tables"].to(gpu), w["scale"], **kw)


def _check(out, w, tol=TOL):
    ref = OA.paged_decode(w["q"].cpu(), w["k_cache"].cpu(), w["v_cache"].cpu(),
                          w["cache_seqlens"].cpu(), w["block_tables"].cpu(), w["scale"])
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= tol, f"max abs err {err}"
    return err


def test_decode_config1_store_then_attend(pkg, gpu):
    """Config 1 end to end: store the new K/V (bit-exact) then attend over ctx+1 keys."""
    w = W.decode_one_layer(seed=0)
    print("[decode] config1", flush=True)
    kc, vc = w["k_cache"].to(gpu), w["v_cache"].to(gpu)
    pkg.kernels.store_kvcache(w["k_new"].to(gpu), w["v_new"].to(gpu), kc, vc,
                              w["slot_mapping"].to(gpu))
    out = pkg.kernels.paged_decode_attention(
        w["q"].to(gpu), kc, vc, w["context_lens"].to(gpu), w["block_tables"].to(gpu),
        w["scale"], seqlen_bias=1)
    torch.cuda.synchronize()
    k_ref, v_ref = w["k_cache"].clone(), w["v_cache"].clone()
    OP.store_kvcache(w["k_new"], w["v_new"], k_ref, v_ref, w["slot_mapping"])
    assert torch.equal(kc.cpu(), k_ref) and torch.equal(vc.cpu(), v_ref)
    w2 = dict(w, k_cache=k_ref, v_cache=v_ref)
    _check(out, w2)
    eager = OA.paged_decode(w["q"], k_ref, v_ref, w["cache_seqlens"], w["block_tables"],
                            w["scale"], mode="bf16_eager")
    assert (out.float().cpu() - eager).abs().max().item() <= TOL


def _ragged(seed, lens, hq=16, hkv=8, extra=3):
    g = torch.Generator().manual_seed(seed)
    need = [max(1, (L + 255) // 256) for L in lens]
    nb = sum(need) + extra
    perm = torch.randperm(nb, generator=g)
    width = max(need)
    bt = torch.full((len(lens), width), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    q = torch.randn(len(lens), hq, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16)
    return dict(q=q, k_cache=kc, v_cache=vc, block_tables=bt,
                cache_seqlens=torch.tensor(lens, dtype=torch.int32), scale=128 ** -0.5)


@pytest.mark.parametrize("pps", [0, 1, 2, 3])
def test_decode_page_boundaries_and_splits(pkg, gpu, pps):
    lens = [1, 2, 255, 256, 257, 511, 512, 513, 1000, 1800]
    w = _ragged(10 + pps, lens)
    print(f"[decode] boundaries pps={pps}", flush=True)
    out = _decode(pkg, gpu, w, pages_per_split=pps)
    torch.cuda.synchronize()
    _check(out, w)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (16, 4), (32, 4)])
def test_decode_gqa_ratios(pkg, gpu, hq, hkv):
    w = _ragged(20 + hq + hkv, [37, 300, 700, 1025], hq=hq, hkv=hkv)
    print(f"[decode] gqa {hq}/{hkv}", flush=True)
    out = _decode(pkg, gpu, w, pages_per_split=1)
    torch.cuda.synchronize()
    _check(out, w)


def test_decode_config3_shape(pkg, gpu):
    """B=64, ctx ~ U{1024..4096}, shuffled tables: the serving-batch shape."""
    w = W.decode_batch(seed=0, batch=64)
    print("[decode] config3 shape", flush=True)
    out = _decode(pkg, gpu, w, seqlen_bias=0)
    torch.cuda.synchronize()
    _check(out, w)


def test_decode_zero_length_gives_zeros_and_strided_q(pkg, gpu):
    w = _ragged(31, [0, 5, 300])
    # q as a strided view of a fused projection: [B, 4096] -> first 2048 = 16 heads.
    g = torch.Generator().manual_seed(32)
    qkv = torch.randn(3, 4096, generator=g).to(torch.bfloat16)
    w["q"] = qkv[:, :2048].view(3, 16, 128)
    print("[decode] zero length + strided q", flush=True)
    out = pkg.kernels.paged_decode_attention(
        qkv.to(gpu)[:, :2048].view(3, 16, 128), w["k_cache"].to(gpu), w["v_cache"].to(gpu),
        w["cache_seqlens"].to(gpu), w["block_tables"].to(gpu), w["scale"])
    torch.cuda.synchronize()
    assert out[0].abs().max().item() == 0.0
    _check(out, w)


def test_decode_graph_replay_matches_eager(pkg, gpu):
    """Capturable: replay with new inputs copied into static buffers."""
    w = _ragged(40, [100, 700, 1300, 260])
    q = w["q"].to(gpu)
    kc, vc = w["k_cache"].to(gpu), w["v_cache"].to(gpu)
    lens = w["cache_seqlens"].to(gpu)
    bt = w["block_tables"].to(gpu)
    print("[decode] graph capture", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.kernels.paged_decode_attention(q, kc, vc, lens, bt, w["scale"])  # warm-up
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.kernels.paged_decode_attention(q, kc, vc, lens, bt, w["scale"])
    g = torch.Generator().manual_seed(41)
    for it in range(4):
        q.copy_(torch.randn(q.shape, generator=g).to(torch.bfloat16))
        lens.copy_(torch.tensor([100 + it * 40, 700 - it, 1300 - 300 * it, 5 + it], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        eager = pkg.kernels.paged_decode_attention(q, kc, vc, lens, bt, w["scale"])
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _check(out, dict(w, q=q.cpu(), cache_seqlens=lens.cpu()))


def test_decode_rejects_bad_shapes(pkg, gpu):
    w = _ragged(50, [10])
    q = w["q"].to(gpu)
    with pytest.raises(ValueError):
        pkg.kernels.paged_decode_attention(q[:, :, :64], w["k_cache"].to(gpu),
                                           w["v_cache"].to(gpu), w["cache_seqlens"].to(gpu),
                                           w["block_tables"].to(gpu), 0.1)
    with pytest.raises(ValueError):
        pkg.kernels.paged_decode_attention(q, w["k_cache"].to(gpu)[:, :128].contiguous(),
                                           w["v_cache"].to(gpu)[:, :128].contiguous(),
                                           w["cache_seqlens"].to(gpu), w["block_tables"].to(gpu),
                                           0.1)


def test_decode_balanced_schedule_ragged_with_empty(pkg, gpu):
    """Balanced schedule: empty sequences in the middle, one-token sequences,
    sequences spanning many workgroups and many sharing one workgroup."""
    lens = [0, 1, 4096, 17, 0, 300, 2049, 1, 255, 256, 257, 3000, 0, 9]
    w = _ragged(60, lens)
    print("[decode] balanced ragged", flush=True)
    out = _decode(pkg, gpu, w)
    torch.cuda.synchronize()
    assert out[0].abs().max().item() == 0.0 and out[4].abs().max().item() == 0.0
    _check(out, w)


def test_decode_balanced_schedule_large_batch(pkg, gpu):
    """More sequences than one workgroup per sequence: 300 short contexts
    (the per-sequence merge), some of them empty."""
    g = torch.Generator().manual_seed(61)
    lens = torch.randint(1, 700, (300,), generator=g).tolist()
    lens[5] = lens[77] = lens[299] = 0
    w = _ragged(62, lens)
    print("[decode] balanced 300 seqs", flush=True)
    out = _decode(pkg, gpu, w)
    torch.cuda.synchronize()
    assert out[[5, 77, 299]].abs().max().item() == 0.0
    _check(out, w)


@pytest.mark.parametrize("hq,hkv", [(2, 2), (8, 2), (4, 4), (16, 4), (8, 8), (32, 8),
                                    (16, 16), (32, 16), (64, 16)])
def test_decode_balanced_schedule_head_layouts(pkg, gpu, hq, hkv):
    """Balanced schedule over every supported KV-head count and GQA ratio
    (the step length is 4 * 16 / Hkv tokens, so each layout cuts pages
    differently); contexts end mid-step, on step and on page boundaries."""
    lens = [1, 7, 8, 9, 63, 64, 65, 255, 256, 257, 700, 1500]
    w = _ragged(70 + hq + hkv, lens, hq=hq, hkv=hkv)
    print(f"[decode] balanced layout {hq}/{hkv}", flush=True)
    out = _decode(pkg, gpu, w)
    torch.cuda.synchronize()
    _check(out, w)


def test_decode_more_than_1024_sequences_uses_split_schedule(pkg, gpu):
    """Beyond 1024 sequences the balanced schedule's in-LDS prefix scan does
    not apply and the per-(sequence, KV head) split takes over."""
    g = torch.Generator().manual_seed(63)
    lens = torch.randint(0, 300, (1100,), generator=g).tolist()
    w = _ragged(64, lens)
    print("[decode] 1100 seqs", flush=True)
    out = _decode(pkg, gpu, w)
    torch.cuda.synchronize()
    _check(out, w)


def test_decode_misaligned_q_view(pkg, gpu):
    """q starting mid-allocation (not 16-byte aligned) is copied by the shim."""
    w = _ragged(33, [40, 300, 700])
    q = w["q"]
    big = torch.zeros(q.numel() + 8, dtype=torch.bfloat16, device=gpu)
    big[1:1 + q.numel()].copy_(q.reshape(-1).to(gpu))
    qm = big[1:1 + q.numel()].view(q.shape)
    print("[decode] misaligned q", flush=True)
    out = pkg.kernels.paged_decode_attention(qm, w["k_cache"].to(gpu), w["v_cache"].to(gpu),
                                             w["cache_seqlens"].to(gpu),
                                             w["block_tables"].to(gpu), w["scale"])
    torch.cuda.synchronize()
    _check(out, w)


def _decode_with_mode(pkg, gpu, w, pps=0):
    """Balanced schedule (``pps`` 0, or -1 for its whole-unit form) through
    the C ABI with an explicit workspace and an output prefilled with 7s;
    returns (out, unit_mode) where unit_mode is the mode word the split
    kernel publishes as the last int32 of its workspace."""
    L = pkg._lib.lib()
    q = w["q"].to(gpu)
    kc, vc = w["k_cache"].to(gpu), w["v_cache"].to(gpu)
    lens = w["cache_seqlens"].to(gpu)
    bt = w["block_tables"].to(gpu)
    bsz, hq, d = q.shape
    nb, _, hkv, _ = kc.shape
    out = torch.full_like(q, 7.0)
    nbytes = L.qmi_paged_decode_workspace_bytes(bsz, hkv, hq, bt.shape[1], pps)
    ws = torch.zeros(nbytes // 4, dtype=torch.int32, device=gpu)
    st = L.qmi_paged_decode_attention(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), nb, 256, hq, hkv,
        d, lens.data_ptr(), 0, bt.data_ptr(), bt.stride(0), bt.shape[1], bsz, w["scale"],
        out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), nbytes, pps,
        torch.cuda.current_stream(gpu).cuda_stream)
    pkg._lib.check(st, "paged_decode_attention")
    torch.cuda.synchronize()
    return out, int(ws[-1].item())


@pytest.mark.parametrize("bsz,hq,hkv", [(256, 16, 8), (128, 16, 8), (256, 16, 4), (300, 32, 16)])
def test_decode_unit_mode_near_equal_lengths(pkg, gpu, bsz, hq, hkv):
    """Batches of 128+ sequences of nearly equal length (a GRPO rollout) run
    one whole (sequence, head group) unit per workgroup with nothing to merge;
    a few empty sequences do not change that."""
    g = torch.Generator().manual_seed(80 + bsz + hkv)
    lens = torch.randint(600, 641, (bsz,), generator=g).tolist()
    lens[3] = lens[bsz - 1] = 0
    w = _ragged(81 + bsz, lens, hq=hq, hkv=hkv)
    print(f"[decode] unit mode B={bsz} {hq}/{hkv}", flush=True)
    out, mode = _decode_with_mode(pkg, gpu, w)
    assert mode == 1
    assert out[[3, bsz - 1]].abs().max().item() == 0.0
    _check(out, w)


@pytest.mark.parametrize("lens_kind,bsz,hq,hkv", [
    ("config1", 4, 16, 8), ("ragged", 64, 16, 8), ("equal", 256, 16, 8), ("ragged", 256, 16, 8),
    ("equal", 128, 16, 4), ("equal", 300, 32, 16), ("empty", 130, 16, 8)])
def test_decode_whole_units_forced(pkg, gpu, lens_kind, bsz, hq, hkv):
    """pages_per_split = -1: one whole (sequence, head group) unit per
    workgroup and no merge launch.  Exact for any lengths (ragged ones only
    balance worse); empty sequences are written as zeros by the split."""
    g = torch.Generator().manual_seed(70 + bsz + hkv)
    if lens_kind == "config1":
        lens = [38, 257, 301, 701]
    elif lens_kind == "equal":
        lens = torch.randint(600, 641, (bsz,), generator=g).tolist()
    elif lens_kind == "empty":
        lens = [0] * bsz
    else:
        lens = torch.randint(1, 1500, (bsz,), generator=g).tolist()
    if lens_kind != "config1":
        lens[1] = lens[bsz - 1] = 0
    w = _ragged(71 + bsz, lens, hq=hq, hkv=hkv)
    print(f"[decode] whole units {lens_kind} B={bsz} {hq}/{hkv}", flush=True)
    out, mode = _decode_with_mode(pkg, gpu, w, pps=-1)
    assert mode == 1
    if lens_kind != "config1":
        assert out[[1, bsz - 1]].abs().max().item() == 0.0
    _check(out, w)


@pytest.mark.parametrize("bsz", [128, 256])
def test_decode_head_group_units_ragged(pkg, gpu, bsz):
    """Ragged lengths at 128+ sequences: the balanced split runs over
    (sequence, head group) units, which then straddle workgroups and merge."""
    g = torch.Generator().manual_seed(90 + bsz)
    lens = torch.randint(1, 1500, (bsz,), generator=g).tolist()
    lens[0] = 0
    w = _ragged(91 + bsz, lens)
    print(f"[decode] head-group units ragged B={bsz}", flush=True)
    out, mode = _decode_with_mode(pkg, gpu, w)
    assert mode == 0
    _check(out, w)


def test_decode_graph_replay_switches_unit_mode(pkg, gpu):
    """One captured graph, replayed with lengths that select unit mode and
    then the balanced split (and back): every replay equals the eager call."""
    bsz = 256
    g = torch.Generator().manual_seed(95)
    w = _ragged(96, [900] * bsz)
    q = w["q"].to(gpu)
    kc, vc = w["k_cache"].to(gpu), w["v_cache"].to(gpu)
    lens = w["cache_seqlens"].to(gpu)
    bt = w["block_tables"].to(gpu)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.kernels.paged_decode_attention(q, kc, vc, lens, bt, w["scale"])
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.kernels.paged_decode_attention(q, kc, vc, lens, bt, w["scale"])
    print("[decode] graph replay across unit mode", flush=True)
    for it, (lo, hi) in enumerate([(880, 900), (1, 900), (700, 720), (0, 400)]):
        new = torch.randint(lo, hi + 1, (bsz,), generator=g, dtype=torch.int32)
        lens.copy_(new)
        q.copy_(torch.randn(q.shape, generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        eager = pkg.kernels.paged_decode_attention(q, kc, vc, lens, bt, w["scale"])
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {it}"
        _check(out, dict(w, q=q.cpu(), cache_seqlens=lens.cpu()))
