"""Pins the oracle's RMSNorm / RoPE restatement (CPU)."""
import torch
import torch.nn.functional as F

from oracle import norm_rope as NR


def test_rms_norm_matches_library():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 1024, generator=g)
    w = torch.randn(1024, generator=g)
    ref = F.rms_norm(x.double(), (1024,), w.double(), eps=1e-6)
    torch.testing.assert_close(NR.rms_norm(x, w).double(), ref, atol=1e-5, rtol=1e-5)


def test_add_rms_norm_residual_and_output():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 64, generator=g).to(torch.bfloat16)
    r = torch.randn(3, 64, generator=g).to(torch.bfloat16)
    w = torch.ones(64)
    out, res = NR.add_rms_norm(x, r, w)
    torch.testing.assert_close(res, (x.float() + r.float()).to(torch.bfloat16))
    ref = F.rms_norm((x.float() + r.float()).double(), (64,), eps=1e-6)
    torch.testing.assert_close(out.double(), ref, atol=2e-2, rtol=1e-2)


def test_rope_matches_complex_rotation():
    g = torch.Generator().manual_seed(2)
    cache = NR.rope_cache(128, 4096, 1e6)
    x = torch.randn(7, 3, 128, generator=g)
    pos = torch.tensor([0, 1, 2, 100, 1000, 4000, 4095])
    out = NR.apply_rope(x, pos, cache, torch.float32)
    ref = NR.apply_rope_complex(x, pos, 128, 1e6)
    torch.testing.assert_close(out.double(), ref, atol=2e-3, rtol=1e-4)


def test_rope_position_zero_identity_and_pair_norms():
    g = torch.Generator().manual_seed(3)
    cache = NR.rope_cache(128, 64, 1e6)
    x = torch.randn(4, 2, 128, generator=g)
    out0 = NR.apply_rope(x, torch.zeros(4, dtype=torch.long), cache, torch.float32)
    torch.testing.assert_close(out0, x)
    pos = torch.tensor([3, 17, 40, 63])
    out = NR.apply_rope(x, pos, cache, torch.float32)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = out[..., :64] ** 2 + out[..., 64:] ** 2
    torch.testing.assert_close(n_out, n_in, atol=1e-4, rtol=1e-5)
