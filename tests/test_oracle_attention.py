"""Pins the oracle's paged decode / varlen prefill attention (CPU).

Independent checks: torch's scaled_dot_product_attention (a library routine)
on contiguous K/V, closed forms (one key, equal keys), chunked == unchunked
prefill and the GQA head mapping.  A transposed operand, a wrong scale, a
wrong causal alignment or a wrong KV-head mapping fails at least one test.
"""
import torch
import torch.nn.functional as F

from oracle import attention as A

D = 128
SCALE = D ** -0.5


def _paged(k_rows, v_rows, num_blocks, page=256, seed=0):
    """Scatter contiguous [L, Hkv, D] rows into a shuffled paged pool."""
    g = torch.Generator().manual_seed(seed)
    L, hkv, d = k_rows.shape
    nblk = (L + page - 1) // page
    perm = torch.randperm(num_blocks, generator=g)[:nblk].tolist()
    kc = torch.randn(num_blocks, page, hkv, d, generator=g)
    vc = torch.randn(num_blocks, page, hkv, d, generator=g)
    for j in range(L):
        kc[perm[j // page], j % page] = k_rows[j]
        vc[perm[j // page], j % page] = v_rows[j]
    return kc, vc, perm


def _sdpa_gqa(q, k, v, causal):
    # q [Lq, Hq, D], k/v [Lk, Hkv, D] -> [Lq, Hq, D] via torch SDPA (fp64).
    rep = q.shape[1] // k.shape[1]
    qq = q.double().permute(1, 0, 2)[None]
    kk = k.double().repeat_interleave(rep, 1).permute(1, 0, 2)[None]
    vv = v.double().repeat_interleave(rep, 1).permute(1, 0, 2)[None]
    if causal and q.shape[0] != k.shape[0]:
        lq, lk = q.shape[0], k.shape[0]
        i = torch.arange(lq)[:, None]
        j = torch.arange(lk)[None, :]
        mask = j <= i + (lk - lq)
        o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=SCALE)
    else:
        o = F.scaled_dot_product_attention(qq, kk, vv, is_causal=causal, scale=SCALE)
    return o[0].permute(1, 0, 2)


def test_decode_matches_sdpa_on_paged_rows():
    g = torch.Generator().manual_seed(1)
    lens = [1, 37, 256, 300, 513]
    kcs, q = [], torch.randn(len(lens), 16, D, generator=g)
    total_blocks = 16
    kc = torch.randn(total_blocks, 256, 8, D, generator=g)
    vc = torch.randn(total_blocks, 256, 8, D, generator=g)
    perm = torch.randperm(total_blocks, generator=g).tolist()
    bt = torch.full((len(lens), 3), -1, dtype=torch.int32)
    off = 0
    for b, L in enumerate(lens):
        n = (L + 255) // 256
        bt[b, :n] = torch.tensor(perm[off:off + n], dtype=torch.int32)
        off += n
    out = A.paged_decode(q, kc, vc, torch.tensor(lens), bt, SCALE, dtype=torch.float64)
    for b, L in enumerate(lens):
        rows = [(int(bt[b, j // 256]), j % 256) for j in range(L)]
        k = torch.stack([kc[p, o] for p, o in rows])
        v = torch.stack([vc[p, o] for p, o in rows])
        ref = _sdpa_gqa(q[b:b + 1], k, v, causal=False)[0]
        torch.testing.assert_close(out[b], ref, atol=1e-10, rtol=1e-10)


def test_decode_single_key_returns_v():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 16, D, generator=g)
    kc = torch.randn(2, 256, 8, D, generator=g)
    vc = torch.randn(2, 256, 8, D, generator=g)
    out = A.paged_decode(q, kc, vc, [1], torch.tensor([[1, 0]]), SCALE, dtype=torch.float64)
    for h in range(16):
        torch.testing.assert_close(out[0, h], vc[1, 0, h // 2].double())


def test_decode_equal_keys_average_v_and_gqa_mapping():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 16, D, generator=g)
    kc = torch.zeros(1, 256, 8, D)
    kc[:] = torch.randn(8, D, generator=g)  # every token has the same keys
    vc = torch.randn(1, 256, 8, D, generator=g)
    out = A.paged_decode(q, kc, vc, [100], torch.tensor([[0]]), SCALE, dtype=torch.float64)
    for h in range(16):
        torch.testing.assert_close(out[0, h], vc[0, :100, h // 2].double().mean(0))
    # Heads 2k and 2k+1 read KV head k; head 2 must not read KV head 0's V.
    assert not torch.allclose(out[0, 2], vc[0, :100, 0].double().mean(0))


def test_prefill_square_is_ordinary_causal():
    g = torch.Generator().manual_seed(4)
    L = 300
    q = torch.randn(L, 16, D, generator=g)
    k = torch.randn(L, 8, D, generator=g)
    v = torch.randn(L, 8, D, generator=g)
    kc, vc, perm = _paged(k, v, 4)
    bt = torch.tensor([perm + [-1] * (4 - len(perm))], dtype=torch.int32)
    out = A.varlen_prefill(q, kc, vc, [0, L], [0, L], bt, SCALE, dtype=torch.float64)
    ref = _sdpa_gqa(q, k, v, causal=True)
    torch.testing.assert_close(out, ref, atol=1e-10, rtol=1e-10)


def test_prefill_bottom_right_alignment_and_chunking():
    # Chunked (prefix cached, then 3 chunks) == unchunked for the same keys:
    # the exact-math form of the reference's chunked-vs-unchunked check
    # (test_chunked_prefill.py:63-155) and of its prefix-cache check.
    g = torch.Generator().manual_seed(5)
    L = 700
    q = torch.randn(L, 16, D, generator=g)
    k = torch.randn(L, 8, D, generator=g)
    v = torch.randn(L, 8, D, generator=g)
    kc, vc, perm = _paged(k, v, 6, seed=9)
    bt = torch.tensor([perm], dtype=torch.int32)
    full = A.varlen_prefill(q, kc, vc, [0, L], [0, L], bt, SCALE, dtype=torch.float64)
    for lo, hi in [(512, 700), (256, 512), (0, 256), (699, 700)]:
        part = A.varlen_prefill(q[lo:hi], kc, vc, [0, hi - lo], [0, hi], bt, SCALE,
                                dtype=torch.float64)
        torch.testing.assert_close(part, full[lo:hi], atol=1e-10, rtol=1e-10)


def test_prefill_varlen_batches_are_independent():
    g = torch.Generator().manual_seed(6)
    kc = torch.randn(8, 256, 8, D, generator=g)
    vc = torch.randn(8, 256, 8, D, generator=g)
    bt = torch.tensor([[2, 5, -1], [7, 0, 3]], dtype=torch.int32)
    q = torch.randn(5 + 9, 16, D, generator=g)
    cu_q, cu_k = [0, 5, 14], [0, 300, 300 + 600]
    out = A.varlen_prefill(q, kc, vc, cu_q, cu_k, bt, SCALE, dtype=torch.float64)
    o0 = A.varlen_prefill(q[:5], kc, vc, [0, 5], [0, 300], bt[:1], SCALE, dtype=torch.float64)
    o1 = A.varlen_prefill(q[5:], kc, vc, [0, 9], [0, 600], bt[1:], SCALE, dtype=torch.float64)
    torch.testing.assert_close(out, torch.cat([o0, o1]))


def test_bf16_eager_mode_close_to_truth():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 16, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(4, 256, 8, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(4, 256, 8, D, generator=g).to(torch.bfloat16)
    bt = torch.tensor([[0, 1], [3, 2]], dtype=torch.int32)
    lens = [300, 41]
    t = A.paged_decode(q, kc, vc, lens, bt, SCALE, mode="fp32")
    e = A.paged_decode(q, kc, vc, lens, bt, SCALE, mode="bf16_eager")
    assert (t - e).abs().max() < 2e-2
