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
ROWS = (1, 7, 64, 65, 100, 129, 200, 256)  # 1, 2, 3 and 4 row tiles of 64, partial ones included


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
