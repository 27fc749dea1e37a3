"""Decode-batch projections (qmi_linear_rows / _parts, qmi_add_rms_norm_parts)
against fp32 torch references of the same products.

Tolerances: the kernels accumulate in fp32 in their own order and round once
to bf16, so outputs agree with the fp32-then-bf16 reference to one bf16 ulp
(relative 2^-8 of the row scale); the SwiGLU epilogue rounds g and u first,
so a one-ulp difference in g moves silu(g) * u by about as much.  The split-K
partial sums are fp32 (1e-5 of the scale), and add_rms_norm_parts is
bit-identical to add_rms_norm on the same bf16 projection output."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

# (K, N) of the Qwen3-0.6B decode projections, plus a small generic one.
SHAPES = {"qkv": (1024, 4096), "o_proj": (2048, 1024), "down": (3072, 1024), "small": (256, 48)}
ROWS = (1, 7, 64, 100, 256)


def _data(gpu, m, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16).to(gpu)
    return x, w


def _rel(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-6)).item()


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("m", ROWS)
def test_linear_rows_plain(pkg, gpu, shape, m):
    k, n = SHAPES[shape]
    x, w = _data(gpu, m, k, n, 11 * m + k)
    print(f"[linear_rows] {shape} m={m}", flush=True)
    y = pkg.kernels.linear_rows(x, w)
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().T).to(torch.bfloat16)
    assert y.shape == (m, n)
    assert _rel(y, ref) <= 1e-2


@pytest.mark.parametrize("m", ROWS)
def test_linear_rows_swiglu(pkg, gpu, m):
    k, inter = 1024, 3072
    x, w = _data(gpu, m, k, 2 * inter, 13 * m)
    print(f"[linear_rows] swiglu m={m}", flush=True)
    y = pkg.kernels.linear_rows(x, w, swiglu=True)
    torch.cuda.synchronize()
    gu = (x.float() @ w.float().T).to(torch.bfloat16)           # the bf16 gate_up output
    ref = pkg.kernels.silu_mul(gu)                                 # then the separate kernel
    g, u = gu.float()[:, :inter], gu.float()[:, inter:]
    ref32 = torch.nn.functional.silu(g) * u
    assert y.shape == (m, inter)
    assert _rel(y, ref32) <= 2e-2
    # Most outputs equal the separate GEMM + silu_mul exactly (same rounding points).
    assert (y == ref).float().mean().item() >= 0.9


@pytest.mark.parametrize("shape", ["o_proj", "down", "small"])
@pytest.mark.parametrize("m", ROWS)
def test_linear_rows_parts_and_norm(pkg, gpu, shape, m):
    k, n = SHAPES[shape]
    x, w = _data(gpu, m, k, n, 17 * m + n)
    g = torch.Generator().manual_seed(m)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16).to(gpu)
    nw = (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16).to(gpu)
    print(f"[linear_rows] parts {shape} m={m}", flush=True)
    p = pkg.kernels.linear_rows_parts(x, w)
    torch.cuda.synchronize()
    n_parts = pkg._lib.lib().qmi_linear_rows_parts_count(m, n, k)
    assert p.parts.shape == (n_parts, m, n)
    ref = x.float() @ w.float().T
    assert _rel(p.parts.sum(0), ref) <= 1e-4
    y, r_out = pkg.kernels.add_rms_norm_parts(p, res, nw, 1e-6)
    # The same sum in the kernel's order (fp32, part 0 first), rounded once.
    acc = p.parts[0].clone()
    for s in range(1, n_parts):
        acc += p.parts[s]
    y_ref, r_ref = pkg.kernels.add_rms_norm(acc.to(torch.bfloat16), res, nw, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(r_out, r_ref)
    assert torch.equal(y, y_ref)


def test_linear_rows_graph_replay(pkg, gpu):
    x, w = _data(gpu, 64, 1024, 4096, 5)
    _, w2 = _data(gpu, 64, 2048, 1024, 6)
    h = torch.randn(64, 2048, device=gpu).to(torch.bfloat16)
    res = torch.randn(64, 1024, device=gpu).to(torch.bfloat16)
    nw = torch.ones(1024, device=gpu, dtype=torch.bfloat16)
    print("[linear_rows] graph capture", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.kernels.linear_rows(x, w)
        pkg.kernels.add_rms_norm_parts(pkg.kernels.linear_rows_parts(h, w2), res, nw, 1e-6)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = pkg.kernels.linear_rows(x, w)
        z, r = pkg.kernels.add_rms_norm_parts(pkg.kernels.linear_rows_parts(h, w2), res, nw, 1e-6)
    g = torch.Generator().manual_seed(9)
    for _ in range(3):
        x.copy_(torch.randn(x.shape, generator=g).to(torch.bfloat16))
        h.copy_(torch.randn(h.shape, generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        y_e = pkg.kernels.linear_rows(x, w)
        z_e, r_e = pkg.kernels.add_rms_norm_parts(pkg.kernels.linear_rows_parts(h, w2), res, nw,
                                                  1e-6)
        torch.cuda.synchronize()
        assert torch.equal(y, y_e) and torch.equal(z, z_e) and torch.equal(r, r_e)


def test_linear_rows_strided_rows(pkg, gpu):
    """x given as a row-strided view (e.g. a slice of a wider buffer)."""
    big = torch.randn(64, 1024 + 256, device=gpu).to(torch.bfloat16)
    x = big[:, :1024]
    _, w = _data(gpu, 64, 1024, 4096, 8)
    print("[linear_rows] strided x", flush=True)
    y = pkg.kernels.linear_rows(x, w)
    ref = (x.float() @ w.float().T).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert _rel(y, ref) <= 1e-2


def test_linear_rows_rejects_bad_shapes(pkg, gpu):
    L = pkg._lib.lib()
    x, w = _data(gpu, 300, 1024, 64, 3)
    y = torch.empty(300, 64, device=gpu, dtype=torch.bfloat16)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.qmi_linear_rows(x.data_ptr(), 1024, w.data_ptr(), 1024, 300, 64, 1024, 0, y.data_ptr(),
                             64, st) != 0                     # more than 256 rows
    assert L.qmi_linear_rows(x.data_ptr(), 1024, w.data_ptr(), 1024, 64, 64, 1000, 0, y.data_ptr(),
                             64, st) != 0                     # K not a multiple of 128
    assert L.qmi_linear_rows(x.data_ptr(), 1024, w.data_ptr(), 1024, 64, 40, 1024, 0, y.data_ptr(),
                             64, st) != 0                     # N not a multiple of 16
    assert L.qmi_linear_rows(x.data_ptr(), 1024, w.data_ptr(), 1024, 64, 64, 1024, 2, y.data_ptr(),
                             64, st) != 0                     # unknown activation
    with pytest.raises(ValueError):
        pkg.kernels.linear_rows(x, w)


@pytest.mark.parametrize("m,hq,hkv", [(1, 16, 8), (7, 16, 8), (64, 16, 8), (100, 16, 8),
                                      (256, 16, 8), (33, 8, 4)])
def test_linear_rows_qk_norm_rope_store(pkg, gpu, m, hq, hkv):
    """qkv projection with the QK-norm / RoPE / KV-store epilogue against (a)
    the same GEMM followed by qk_norm_rope_store (same bf16 projection output:
    v rows bit-identical, q and k within one ulp, since only the fp32 order of
    the head's sum of squares differs) and (b) the oracle's norm and rotation
    of that output (2 ulps: two roundings in the chain).  Slots -1 and past
    the pool are skipped; untouched cache rows keep their contents."""
    from oracle import norm_rope as NR

    k = 1024
    n = (hq + 2 * hkv) * 128
    x, w = _data(gpu, m, k, n, 17 * m + hq)
    g = torch.Generator().manual_seed(m)
    qw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(gpu)
    kw = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16).to(gpu)
    pos = torch.randint(0, 40960, (m,), generator=g)
    pos[0] = 0
    nb = (m + 255) // 256 + 1
    slots = torch.randperm(nb * 256, generator=g)[:m].to(torch.int32)
    if m > 8:
        slots[3], slots[7] = -1, nb * 256 + 5
    cache = NR.rope_cache(128, 40960, 1e6).to(gpu)
    base_k = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16).to(gpu)
    base_v = torch.randn(nb, 256, hkv, 128, generator=g).to(torch.bfloat16).to(gpu)
    print(f"[linear_rows] qkv + qk-norm/rope/store m={m} hq={hq} hkv={hkv}", flush=True)
    k1, v1 = base_k.clone(), base_v.clone()
    qkv = pkg.kernels.linear_rows(x, w)
    q1 = pkg.kernels.qk_norm_rope_store(qkv, qw, kw, pos.to(gpu), cache, hq, hkv, 1e-6, k1, v1,
                                        slots.to(gpu))
    k2, v2 = base_k.clone(), base_v.clone()
    q2 = pkg.kernels.linear_rows_qk_norm_rope_store(x, w, qw, kw, pos.to(gpu), cache, hq, hkv,
                                                    1e-6, k2, v2, slots.to(gpu))
    torch.cuda.synchronize()
    assert q2.shape == (m, hq, 128)
    assert torch.equal(v1, v2)
    ok = slots.long()
    ok = ok[(ok >= 0) & (ok < nb * 256)]
    untouched = torch.ones(nb * 256, dtype=torch.bool)
    untouched[ok] = False
    assert torch.equal(k2.view(-1, hkv, 128)[untouched.to(gpu)],
                       base_k.view(-1, hkv, 128)[untouched.to(gpu)])
    # A one-ulp flip of a normalised value moves the rotated pair by one ulp
    # of the larger partner, so the bound adds one ulp of the head row's scale.
    for a, b in ((q1, q2), (k1, k2)):
        d = (a.float() - b.float()).abs()
        bf = b.float()
        tol = 2.0 ** -7 * (bf.abs() + bf.abs().amax(-1, keepdim=True)) + 1e-30
        assert (d > tol).sum().item() == 0
        assert (a == b).float().mean().item() >= 0.99
    # Against the oracle's norm + rotation of the bf16 projection output.
    qkv_c = qkv.cpu()
    qn = NR.rms_norm(qkv_c[:, :hq * 128].view(m, hq, 128), qw.cpu(), 1e-6)
    kn = NR.rms_norm(qkv_c[:, hq * 128:(hq + hkv) * 128].view(m, hkv, 128), kw.cpu(), 1e-6)
    rq = NR.apply_rope(qn, pos, cache.cpu(), torch.bfloat16)
    rk = NR.apply_rope(kn, pos, cache.cpu(), torch.bfloat16)
    got_k = k2.cpu().view(-1, hkv, 128)
    sel = slots.long()
    valid = (sel >= 0) & (sel < nb * 256)
    for got, ref in ((q2.cpu(), rq), (got_k[sel[valid]], rk[valid])):
        d = (got.float() - ref.float()).abs()
        rf = ref.float().abs()
        tol = 2.0 ** -7 * (2 * rf + rf.amax(-1, keepdim=True)) + 1e-30
        assert (d > tol).sum().item() == 0, f"max diff {d.max().item()}"
    assert torch.equal(q2[0].cpu(), qn[0])  # position 0: the rotation is the identity
    v_ref = qkv_c[:, (hq + hkv) * 128:].view(m, hkv, 128)
    assert torch.equal(v2.cpu().view(-1, hkv, 128)[sel[valid]], v_ref[valid])
