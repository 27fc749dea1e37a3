"""qmi_paged_decode_attention_noalloc (no allocation: a static device array
as the workspace) against qmi_paged_decode_attention (caller workspace),
both called through the C ABI: two calls in a row, the second with a
smaller problem, must give bit-identical outputs; a problem beyond the
static array's size is rejected before anything is launched."""
import pytest
import torch

from oracle import workloads as W

pytestmark = pytest.mark.gpu

SCRATCH_LIMIT = -6


def _args(w, out):
    q, kc, lens, bt = w["q"], w["k_cache"], w["cache_seqlens"], w["block_tables"]
    bsz, hq, d = q.shape
    return (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), w["v_cache"].data_ptr(),
            kc.shape[0], 256, hq, kc.shape[2], d, lens.data_ptr(), 0, bt.data_ptr(),
            bt.stride(0), bt.shape[1], bsz, float(w["scale"]), out.data_ptr(), out.stride(0),
            out.stride(1))


def _regular(L, w, pps, stream):
    out = torch.full_like(w["q"], float("nan"))
    q, kc = w["q"], w["k_cache"]
    nbytes = L.qmi_paged_decode_workspace_bytes(q.shape[0], kc.shape[2], q.shape[1],
                                                w["block_tables"].shape[1], pps)
    ws = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=q.device)
    st = L.qmi_paged_decode_attention(*_args(w, out), ws.data_ptr(), nbytes, pps, stream)
    assert st == 0, L.qmi_error_string(st)
    return out


def _noalloc(L, w, pps, stream):
    out = torch.full_like(w["q"], float("nan"))
    st = L.qmi_paged_decode_attention_noalloc(*_args(w, out), pps, stream)
    assert st == 0, L.qmi_error_string(st)
    return out


@pytest.mark.parametrize("pps", [0, -1, 2])
def test_noalloc_matches_workspace_entry(pkg, gpu, pps):
    L = pkg._lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    big = W.decode_batch(seed=0, device=gpu, batch=64)                    # config 3, one layer
    small = W.decode_batch(seed=5, device=gpu, batch=9, ctx_lo=0, ctx_hi=700)
    for name, w in (("B=64 ctx U{1024..4096}", big), ("B=9 ctx U{0..700}", small)):
        print(f"[noalloc] pages_per_split={pps} {name}", flush=True)
        ref = _regular(L, w, pps, stream)
        got = _noalloc(L, w, pps, stream)
        torch.cuda.synchronize()
        assert not torch.isnan(ref.float()).any()
        assert torch.equal(got, ref)


def test_noalloc_rejects_problems_beyond_the_scratch(pkg, gpu):
    """16 KV heads x 4 query heads each need 34.6 MB of balanced-split
    partials on 256 CUs: more than the 16 MiB array, so the call returns
    QMI_E_SCRATCH_LIMIT without launching."""
    L = pkg._lib.lib()
    w = W.decode_batch(seed=1, device=gpu, batch=4, ctx_lo=10, ctx_hi=20)
    q = torch.zeros((4, 64, 128), dtype=torch.bfloat16, device=gpu)
    kc = torch.zeros((w["num_blocks"], 256, 16, 128), dtype=torch.bfloat16, device=gpu)
    w2 = dict(w, q=q, k_cache=kc, v_cache=kc)
    out = torch.zeros_like(q)
    need = L.qmi_paged_decode_workspace_bytes(4, 16, 64, w["block_tables"].shape[1], 0)
    print(f"[noalloc] 64/16 heads need {need} B", flush=True)
    assert need > 16 << 20
    assert L.qmi_paged_decode_attention_noalloc(*_args(w2, out), 0,
                                                torch.cuda.current_stream().cuda_stream) == SCRATCH_LIMIT
    assert b"static device scratch" in L.qmi_error_string(SCRATCH_LIMIT)


def test_noalloc_balanced_schedule_with_graph_width_tables(pkg, gpu):
    """256 sequences with page tables padded to 160 entries (the engine's
    graph width): the balanced schedule needs 8.7 MB, within the array, even
    though the per-split schedule of the same shape would need 34.6 MB."""
    L = pkg._lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    w = W.decode_batch(seed=7, device=gpu, batch=256, ctx_lo=100, ctx_hi=1100)
    bt = torch.full((256, 160), -1, dtype=torch.int32, device=gpu)
    bt[:, :w["block_tables"].shape[1]] = w["block_tables"]
    w = dict(w, block_tables=bt)
    print("[noalloc] B=256, table width 160", flush=True)
    ref = _regular(L, w, 0, stream)
    got = _noalloc(L, w, 0, stream)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
