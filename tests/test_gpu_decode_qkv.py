"""Decode attention with the QK-norm / RoPE / KV store folded in
(qmi_paged_decode_attention_qkv) against

  (a) the two-call form it replaces, qk_norm_rope_store + paged decode
      attention (bias 1) on the same inputs: V cache rows bit-identical,
      untouched cache rows unchanged, outputs within 1e-2, and the written K
      rows within the bound that one bf16 ulp in each normalised input of
      the rotation allows (only the fp32 order of each head's sum of squares
      differs, which can move a rounded norm output by one ulp; the rotation
      n1 c - n2 s can cancel, so the bound is 2^-7 (|n1 c| + |n2 s| + |o|)
      per element, not one ulp of the output);
  (b) the oracle: norm + RoPE (oracle.norm_rope), the slot store
      (oracle.paged.store_kvcache) and fp32 decode attention
      (oracle.attention.paged_decode), outputs within 2e-2 and the written K
      rows within the same bound.

Cases: the config-1 shape, ragged batches that take the balanced split with
partial slots and its merge, near-equal batches that take one whole unit per
workgroup (detected on the device, and forced with pages_per_split=-1), new
tokens at the first and last row of a page, slot -1 rows, GQA layouts."""
import pytest
import torch

from oracle import attention as OA
from oracle import norm_rope as NR
from oracle import paged as OP

pytestmark = pytest.mark.gpu

TOL = 2e-2
MAXPOS = 8192


def _case(seed, ctx, hq=16, hkv=8, extra=2, skip=()):
    """Random qkv rows, pools and tables for decode with context lengths ctx
    (the new token of sequence b is key ctx[b], stored at its table slot)."""
    g = torch.Generator().manual_seed(seed)
    need = [(c + 1 + 255) // 256 for c in ctx]
    nb = sum(need) + extra
    perm = torch.randperm(nb, generator=g)
    width = max(need)
    bt = torch.full((len(ctx), width), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    slots = torch.tensor([OP.decode_slot(bt[b, :need[b]].tolist(), c) for b, c in enumerate(ctx)],
                         dtype=torch.int32)
    for b in skip:
        slots[b] = -1
    qkv = (torch.randn(len(ctx), (hq + 2 * hkv) * 128, generator=g) * 2).to(torch.bfloat16)
    kc = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16)
    qw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    return dict(qkv=qkv, k_cache=kc, v_cache=vc, block_tables=bt, slots=slots, qw=qw, kw=kw,
                ctx=torch.tensor(ctx, dtype=torch.int32), pos=torch.tensor(ctx, dtype=torch.int64),
                hq=hq, hkv=hkv, scale=128 ** -0.5)


def _run_both(pkg, gpu, w, pps):
    K = pkg.kernels
    cache = NR.rope_cache(128, MAXPOS, 1e6).to(gpu)
    dev = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    k1, v1 = dev["k_cache"].clone(), dev["v_cache"].clone()
    q = K.qk_norm_rope_store(dev["qkv"], dev["qw"], dev["kw"], dev["pos"], cache, w["hq"],
                             w["hkv"], 1e-6, k1, v1, dev["slots"])
    o1 = K.paged_decode_attention(q, k1, v1, dev["ctx"], dev["block_tables"], w["scale"],
                                  seqlen_bias=1, pages_per_split=pps)
    k2, v2 = dev["k_cache"].clone(), dev["v_cache"].clone()
    o2 = K.paged_decode_attention_qkv(dev["qkv"], dev["qw"], dev["kw"], dev["pos"], cache,
                                      w["hq"], w["hkv"], 1e-6, k2, v2, dev["slots"], dev["ctx"],
                                      dev["block_tables"], w["scale"], pages_per_split=pps)
    torch.cuda.synchronize()
    return o1, k1, v1, o2, k2, v2


def _rope_bound(w, rows):
    """Per-element bound of the written K rows of sequences ``rows``: one bf16
    ulp (<= 2^-7 |x|) in each normalised input of o1 = n1 c - n2 s,
    o2 = n2 c + n1 s, plus the two outputs' own roundings."""
    hq, hkv = w["hq"], w["hkv"]
    raw = w["qkv"][rows].view(len(rows), hq + 2 * hkv, 128)[:, hq:hq + hkv]
    n = NR.rms_norm(raw, w["kw"]).float()
    cs = NR.rope_cache(128, MAXPOS, 1e6)[w["pos"][rows]]
    c, s = cs[:, None, :64].abs(), cs[:, None, 64:].abs()
    n1, n2 = n[..., :64].abs(), n[..., 64:].abs()
    mag = torch.cat((n1 * c + n2 * s, n2 * c + n1 * s), dim=-1)
    o = NR.apply_rope(NR.rms_norm(raw, w["kw"]), w["pos"][rows],
                      NR.rope_cache(128, MAXPOS, 1e6)).float()
    return 2.0 ** -7 * (mag + o.abs()) + 1e-30


def _k_close(w, got, ref):
    """Written K rows (by slot order of the stored sequences) within the bound."""
    rows = [b for b in range(len(w["slots"])) if int(w["slots"][b]) >= 0]
    if not rows:
        return
    tol = _rope_bound(w, rows)
    slots = [int(w["slots"][b]) for b in rows]
    hkv = w["hkv"]
    a = got.view(-1, hkv, 128).cpu()[slots].float()
    b = ref.view(-1, hkv, 128).cpu()[slots].float()
    bad = ((a - b).abs() > tol).sum().item()
    assert bad == 0, f"{bad} K elements beyond the bound (max diff {(a - b).abs().max().item()})"


def _compare(w, o1, k1, v1, o2, k2, v2):
    assert torch.equal(v1, v2), "V cache differs from the two-call form"
    hkv = w["hkv"]
    written = [int(s) for s in w["slots"] if int(s) >= 0]
    kf1 = k1.view(-1, hkv, 128).cpu()
    kf2 = k2.view(-1, hkv, 128).cpu()
    mask = torch.ones(kf1.shape[0], dtype=torch.bool)
    mask[written] = False
    assert torch.equal(kf1[mask], kf2[mask]), "rows outside the new slots changed"
    _k_close(w, k2, k1)
    err = (o1.float() - o2.float()).abs().max().item()
    assert err <= 1e-2, f"fused vs two-call max abs diff {err}"
    return err


def _oracle_check(w, o2, k2):
    """The oracle's store-then-attend on the CPU."""
    hq, hkv = w["hq"], w["hkv"]
    n = w["qkv"].shape[0]
    qkv = w["qkv"].view(n, hq + 2 * hkv, 128)
    cache = NR.rope_cache(128, MAXPOS, 1e6)
    q = NR.apply_rope(NR.rms_norm(qkv[:, :hq], w["qw"]), w["pos"], cache)
    k = NR.apply_rope(NR.rms_norm(qkv[:, hq:hq + hkv], w["kw"]), w["pos"], cache)
    v = qkv[:, hq + hkv:].contiguous()
    kr, vr = w["k_cache"].clone(), w["v_cache"].clone()
    OP.store_kvcache(k, v, kr, vr, w["slots"])
    _k_close(w, k2, kr)
    ref = OA.paged_decode(q, kr, vr, w["ctx"] + 1, w["block_tables"], w["scale"])
    err = (o2.float().cpu() - ref).abs().max().item()
    assert err <= TOL, f"fused vs oracle max abs err {err}"


def test_qkv_decode_config1_shape(pkg, gpu):
    """Config 1: 4 sequences, contexts 37 / 256 / 300 / 700, 16-page pool."""
    w = _case(1, [37, 256, 300, 700], extra=16 - 7)
    print("[decode_qkv] config1 shape", flush=True)
    res = _run_both(pkg, gpu, w, 0)
    _compare(w, *res)
    _oracle_check(w, res[3], res[4])


@pytest.mark.parametrize("pps", [0, -1])
def test_qkv_decode_page_edges_and_skips(pkg, gpu, pps):
    """New tokens at the first / last row of a page, contexts 0 and 1, and
    rows with slot -1 (not stored; key ctx read from the cache as it is)."""
    ctx = [0, 1, 254, 255, 256, 511, 512, 767, 1000, 1023, 1024, 3]
    w = _case(2 + pps, ctx, skip=(3, 9))
    print(f"[decode_qkv] page edges pps={pps}", flush=True)
    res = _run_both(pkg, gpu, w, pps)
    _compare(w, *res)
    _oracle_check(w, res[3], res[4])


@pytest.mark.parametrize("batch,lo,hi", [(64, 1, 2000), (200, 100, 900), (256, 600, 680),
                                         (256, 128, 1152)])
def test_qkv_decode_batches(pkg, gpu, batch, lo, hi):
    """Ragged batches (balanced split, partial slots, merge) and near-equal
    batches of 256 (head-group units, one whole unit per workgroup)."""
    g = torch.Generator().manual_seed(batch + lo)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=g).tolist()
    w = _case(batch + hi, ctx)
    print(f"[decode_qkv] batch={batch} ctx U{{{lo}..{hi}}}", flush=True)
    res = _run_both(pkg, gpu, w, 0)
    _compare(w, *res)
    # The oracle on a sample of sequences (fp32 CPU attention is slow).
    idx = list(range(0, batch, max(1, batch // 6)))[:6]
    sub = dict(w, qkv=w["qkv"][idx], block_tables=w["block_tables"][idx], slots=w["slots"][idx],
               ctx=w["ctx"][idx], pos=w["pos"][idx])
    ref_out = res[3][idx]
    _oracle_check(sub, ref_out, res[4])


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 4), (32, 8), (8, 2)])
def test_qkv_decode_gqa_layouts(pkg, gpu, hq, hkv):
    w = _case(hq * 10 + hkv, [5, 300, 700, 1025, 2000], hq=hq, hkv=hkv)
    print(f"[decode_qkv] hq={hq} hkv={hkv}", flush=True)
    res = _run_both(pkg, gpu, w, 0)
    _compare(w, *res)
    _oracle_check(w, res[3], res[4])


def test_qkv_decode_graph_replay(pkg, gpu):
    """Captured once, replayed with new contexts written into the same
    buffers: every replay equals the eager call on the same inputs."""
    K = pkg.kernels
    ctx0 = [100, 900, 1500, 40, 2047, 511]
    w = _case(7, [c + 8 for c in ctx0])  # tables wide enough for every replay
    cache = NR.rope_cache(128, MAXPOS, 1e6).to(gpu)
    dev = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    ctx_buf = torch.tensor(ctx0, dtype=torch.int32, device=gpu)
    pos_buf = ctx_buf.long()
    slot_buf = torch.zeros(len(ctx0), dtype=torch.int32, device=gpu)
    kc, vc = dev["k_cache"].clone(), dev["v_cache"].clone()
    out = torch.empty(len(ctx0), w["hq"], 128, dtype=torch.bfloat16, device=gpu)
    bt_cpu = w["block_tables"]

    def fill(step):
        c = [x + step for x in ctx0]
        ctx_buf.copy_(torch.tensor(c, dtype=torch.int32))
        pos_buf.copy_(torch.tensor(c, dtype=torch.int64))
        slot_buf.copy_(torch.tensor([OP.decode_slot(bt_cpu[b].tolist(), x)
                                     for b, x in enumerate(c)], dtype=torch.int32))

    def call():
        K.paged_decode_attention_qkv(dev["qkv"], dev["qw"], dev["kw"], pos_buf, cache, w["hq"],
                                     w["hkv"], 1e-6, kc, vc, slot_buf, ctx_buf,
                                     dev["block_tables"], w["scale"], out=out)

    print("[decode_qkv] graph replay", flush=True)
    fill(0)
    call()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.synchronize()
    for step in range(1, 5):
        fill(step)
        kref, vref = kc.clone(), vc.clone()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        got_k, got_v = kc.clone(), vc.clone()
        kc.copy_(kref)
        vc.copy_(vref)
        call()
        torch.cuda.synchronize()
        assert torch.equal(got, out) and torch.equal(got_k, kc) and torch.equal(got_v, vc)


def test_qkv_decode_rejects_bad_arguments(pkg, gpu):
    K = pkg.kernels
    w = _case(3, [10, 20])
    cache = NR.rope_cache(128, MAXPOS, 1e6).to(gpu)
    dev = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    args = (dev["qw"], dev["kw"], dev["pos"], cache, w["hq"], w["hkv"], 1e-6, dev["k_cache"],
            dev["v_cache"], dev["slots"], dev["ctx"], dev["block_tables"], w["scale"])
    with pytest.raises(ValueError):
        K.paged_decode_attention_qkv(dev["qkv"][:, :-128], *args)        # wrong row width
    with pytest.raises(ValueError):
        K.paged_decode_attention_qkv(dev["qkv"], *args, pages_per_split=2)
    bad = list(args)
    bad[2] = w["pos"]                                                     # host positions
    with pytest.raises(ValueError):
        K.paged_decode_attention_qkv(dev["qkv"], *bad)
    L = pkg._lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    p = dev["qkv"]
    ws = torch.empty(1 << 18, dtype=torch.float32, device=gpu)
    out = torch.empty(2, 16, 128, dtype=torch.bfloat16, device=gpu)
    # head_dim 64 is unsupported; a null slot mapping is rejected
    assert L.qmi_paged_decode_attention_qkv(
        p.data_ptr(), p.stride(0), 16, 8, 64, dev["qw"].data_ptr(), dev["kw"].data_ptr(),
        dev["pos"].data_ptr(), cache.data_ptr(), MAXPOS, 1e-6, dev["k_cache"].data_ptr(),
        dev["v_cache"].data_ptr(), dev["k_cache"].shape[0], 256, dev["slots"].data_ptr(),
        dev["ctx"].data_ptr(), dev["block_tables"].data_ptr(), dev["block_tables"].stride(0),
        dev["block_tables"].shape[1], 2, w["scale"], out.data_ptr(), 2048, 128, ws.data_ptr(),
        1 << 20, 0, st) != 0
    assert L.qmi_paged_decode_attention_qkv(
        p.data_ptr(), p.stride(0), 16, 8, 128, dev["qw"].data_ptr(), dev["kw"].data_ptr(),
        dev["pos"].data_ptr(), cache.data_ptr(), MAXPOS, 1e-6, dev["k_cache"].data_ptr(),
        dev["v_cache"].data_ptr(), dev["k_cache"].shape[0], 256, None,
        dev["ctx"].data_ptr(), dev["block_tables"].data_ptr(), dev["block_tables"].stride(0),
        dev["block_tables"].shape[1], 2, w["scale"], out.data_ptr(), 2048, 128, ws.data_ptr(),
        1 << 20, 0, st) != 0
