"""RMSNorm / add+RMSNorm / fused QK-norm+RoPE / SwiGLU kernels against the
oracle.  Outputs are bf16; the tolerance is one bf16 ulp of the value (the
kernels compute in fp32 with a different summation order)."""
import pytest
import torch

from oracle import norm_rope as NR

pytestmark = pytest.mark.gpu


def ulp_close(a, b, ulps=1.0):
    a = a.float().cpu()
    b = b.float().cpu()
    tol = ulps * 2.0 ** -7 * b.abs().clamp_min(2.0 ** -100) + 1e-30
    bad = ((a - b).abs() > tol).sum().item()
    return bad == 0, bad, (a - b).abs().max().item()


@pytest.mark.parametrize("n", [128, 1024, 3072])
def test_rms_norm(pkg, gpu, n):
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(37, n, generator=g) * 3).to(torch.bfloat16)
    w = (torch.rand(n, generator=g) + 0.5).to(torch.bfloat16)
    print(f"[norm] rms n={n}", flush=True)
    y = pkg.kernels.rms_norm(x.to(gpu), w.to(gpu), 1e-6)
    torch.cuda.synchronize()
    ok, bad, mx = ulp_close(y, NR.rms_norm(x, w, 1e-6))
    assert ok, f"{bad} elements beyond 1 ulp (max diff {mx})"


def test_add_rms_norm(pkg, gpu):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    r = torch.randn(64, 1024, generator=g).to(torch.bfloat16)
    w = (torch.rand(1024, generator=g) + 0.5).to(torch.bfloat16)
    print("[norm] add+rms", flush=True)
    y, res = pkg.kernels.add_rms_norm(x.to(gpu), r.to(gpu), w.to(gpu), 1e-6)
    torch.cuda.synchronize()
    ry, rres = NR.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(res.cpu(), rres)          # bf16(x + r): exact
    ok, bad, mx = ulp_close(y, ry)
    assert ok, f"{bad} elements beyond 1 ulp (max diff {mx})"


def test_qk_norm_rope(pkg, gpu):
    g = torch.Generator().manual_seed(2)
    n, hq, hkv = 50, 16, 8
    qkv = (torch.randn(n, (hq + 2 * hkv) * 128, generator=g) * 2).to(torch.bfloat16)
    qw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, 40960, (n,), generator=g)
    pos[0] = 0
    cache = NR.rope_cache(128, 40960, 1e6)
    print("[norm] qk norm + rope", flush=True)
    q, k = pkg.kernels.qk_norm_rope(qkv.to(gpu), qw.to(gpu), kw.to(gpu), pos.to(gpu),
                                    cache.to(gpu), hq, hkv, 1e-6)
    torch.cuda.synchronize()
    qn = NR.rms_norm(qkv[:, :hq * 128].view(n, hq, 128), qw, 1e-6)
    kn = NR.rms_norm(qkv[:, hq * 128:(hq + hkv) * 128].view(n, hkv, 128), kw, 1e-6)
    rq = NR.apply_rope(qn, pos, cache, torch.bfloat16)
    rk = NR.apply_rope(kn, pos, cache, torch.bfloat16)
    # Two roundings in the chain (norm output, rope output): allow 2 ulps.
    for got, ref in ((q, rq), (k, rk)):
        ok, bad, mx = ulp_close(got, ref, 2.0)
        assert ok, f"{bad} elements beyond 2 ulp (max diff {mx})"
    assert torch.equal(q[0].cpu(), qn[0])        # position 0 rotates by identity


def test_qk_norm_rope_store_equals_separate_kernels(pkg, gpu):
    """The fused store writes exactly what qk_norm_rope + store_kvcache write
    (bit-identical q, K and V rows); slots -1 and past the pool are skipped."""
    g = torch.Generator().manual_seed(3)
    n, hq, hkv, nb = 40, 16, 8, 3
    qkv = (torch.randn(n, (hq + 2 * hkv) * 128, generator=g) * 2).to(torch.bfloat16).to(gpu)
    qw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(gpu)
    kw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(gpu)
    pos = torch.randint(0, 4096, (n,), generator=g).to(gpu)
    slots = torch.randperm(nb * 256, generator=g)[:n].to(torch.int32)
    slots[3], slots[7] = -1, nb * 256 + 5
    slots = slots.to(gpu)
    cache = NR.rope_cache(128, 40960, 1e6).to(gpu)
    base_k = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16).to(gpu)
    base_v = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16).to(gpu)
    print("[norm] qk norm + rope + store", flush=True)
    k1, v1 = base_k.clone(), base_v.clone()
    q1, kk = pkg.kernels.qk_norm_rope(qkv, qw, kw, pos, cache, hq, hkv, 1e-6)
    vv = qkv[:, (hq + hkv) * 128:].view(n, hkv, 128)
    pkg.kernels.store_kvcache(kk, vv, k1, v1, slots)
    k2, v2 = base_k.clone(), base_v.clone()
    q2 = pkg.kernels.qk_norm_rope_store(qkv, qw, kw, pos, cache, hq, hkv, 1e-6, k2, v2, slots)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert not torch.equal(k2, base_k)


def test_silu_mul(pkg, gpu):
    g = torch.Generator().manual_seed(3)
    gu = (torch.randn(33, 2 * 3072, generator=g) * 2).to(torch.bfloat16)
    print("[norm] silu*mul", flush=True)
    out = pkg.kernels.silu_mul(gu.to(gpu))
    torch.cuda.synchronize()
    gf, uf = gu[:, :3072].float(), gu[:, 3072:].float()
    ref = (torch.nn.functional.silu(gf) * uf).to(torch.bfloat16)
    ok, bad, mx = ulp_close(out, ref, 1.0)
    assert ok, f"{bad} elements beyond 1 ulp (max diff {mx})"


@pytest.mark.parametrize("n,hq,hkv", [(7, 16, 8), (5, 8, 4), (1, 16, 8), (3, 4, 4)])
def test_qk_norm_rope_store_partial_workgroups(pkg, gpu, n, hq, hkv):
    """Token x head counts that leave the last workgroup (16 heads) partly
    empty; other GQA ratios; every token stored."""
    g = torch.Generator().manual_seed(20 + n + hq)
    nb = 2
    qkv = (torch.randn(n, (hq + 2 * hkv) * 128, generator=g) * 2).to(torch.bfloat16)
    qw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, 40960, (n,), generator=g)
    slots = torch.randperm(nb * 256, generator=g)[:n].to(torch.int32)
    cache = NR.rope_cache(128, 40960, 1e6)
    kc = torch.zeros(nb, 256, hkv, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    print(f"[norm] partial workgroups n={n} hq={hq} hkv={hkv}", flush=True)
    kcg, vcg = kc.to(gpu), vc.to(gpu)
    q = pkg.kernels.qk_norm_rope_store(qkv.to(gpu), qw.to(gpu), kw.to(gpu), pos.to(gpu),
                                       cache.to(gpu), hq, hkv, 1e-6, kcg, vcg, slots.to(gpu))
    torch.cuda.synchronize()
    qn = NR.rms_norm(qkv[:, :hq * 128].view(n, hq, 128), qw, 1e-6)
    kn = NR.rms_norm(qkv[:, hq * 128:(hq + hkv) * 128].view(n, hkv, 128), kw, 1e-6)
    rq = NR.apply_rope(qn, pos, cache, torch.bfloat16)
    rk = NR.apply_rope(kn, pos, cache, torch.bfloat16)
    ok, bad, mx = ulp_close(q, rq, 2.0)
    assert ok, f"q: {bad} elements beyond 2 ulp (max diff {mx})"
    got_k = kcg.cpu().view(-1, hkv, 128)[slots.long()]
    ok, bad, mx = ulp_close(got_k, rk, 2.0)
    assert ok, f"k: {bad} elements beyond 2 ulp (max diff {mx})"
    v = qkv[:, (hq + hkv) * 128:].view(n, hkv, 128)
    assert torch.equal(vcg.cpu().view(-1, hkv, 128)[slots.long()], v)


def test_qk_norm_rope_misaligned_rows(pkg, gpu):
    """The kernel reads rows 8 / 16 bytes at a time: through the C ABI a qkv
    view starting one element into its storage is rejected (not read
    unaligned); the Python wrapper copies it and gives the aligned result."""
    import ctypes
    n, hq, hkv = 4, 16, 8
    row = (hq + 2 * hkv) * 128
    g = torch.Generator().manual_seed(30)
    src = torch.randn(n, row, generator=g).to(torch.bfloat16).to(gpu)
    big = torch.zeros(n * row + 8, dtype=torch.bfloat16, device=gpu)
    big[1:1 + n * row].copy_(src.reshape(-1))
    qkv = big[1:1 + n * row].view(n, row)
    w = torch.ones(128, dtype=torch.bfloat16, device=gpu)
    pos = torch.arange(n, dtype=torch.int64, device=gpu)
    cache = NR.rope_cache(128, 64, 1e6).to(gpu)
    print("[norm] misaligned qkv rows", flush=True)
    q_ref, k_ref = pkg.kernels.qk_norm_rope(src, w, w, pos, cache, hq, hkv, 1e-6)
    q, k = pkg.kernels.qk_norm_rope(qkv, w, w, pos, cache, hq, hkv, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref) and torch.equal(k, k_ref)
    q_out = torch.empty(n, hq, 128, dtype=torch.bfloat16, device=gpu)
    k_out = torch.empty(n, hkv, 128, dtype=torch.bfloat16, device=gpu)
    st = pkg._lib.lib().qmi_qk_norm_rope(
        qkv.data_ptr(), qkv.stride(0), n, hq, hkv, 128, w.data_ptr(), w.data_ptr(), pos.data_ptr(),
        cache.data_ptr(), cache.shape[0], q_out.data_ptr(), q_out.stride(0), k_out.data_ptr(),
        k_out.stride(0), 1e-6, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st != 0


def test_body_kernels_accept_misaligned_views(pkg, gpu):
    """Rows starting mid-allocation (not 16-byte aligned) are copied by the
    shims and give the same result as aligned rows."""
    g = torch.Generator().manual_seed(31)
    x = torch.randn(6, 1024, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.rand(1024, generator=g) + 0.5).to(torch.bfloat16).to(gpu)
    big = torch.zeros(6 * 1024 + 8, dtype=torch.bfloat16, device=gpu)
    big[3:3 + 6 * 1024].copy_(x.reshape(-1))
    xm = big[3:3 + 6 * 1024].view(6, 1024)
    print("[norm] misaligned rows", flush=True)
    assert torch.equal(pkg.kernels.rms_norm(xm, w, 1e-6), pkg.kernels.rms_norm(x, w, 1e-6))
    gu = torch.randn(6, 2 * 1024, generator=g).to(torch.bfloat16).to(gpu)
    big2 = torch.zeros(6 * 2048 + 8, dtype=torch.bfloat16, device=gpu)
    big2[5:5 + 6 * 2048].copy_(gu.reshape(-1))
    assert torch.equal(pkg.kernels.silu_mul(big2[5:5 + 6 * 2048].view(6, 2048)), pkg.kernels.silu_mul(gu))
