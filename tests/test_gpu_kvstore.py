"""KV store parity: the HIP slot-mapped store is bit-exact with the oracle."""
import pytest
import torch

from oracle import paged as OP
from oracle import workloads as W

pytestmark = pytest.mark.gpu


def _run_both(pkg, gpu, key, value, kc, vc, slots):
    print(f"[store] N={key.shape[0]} cache={tuple(kc.shape)}", flush=True)
    k_ref, v_ref = kc.clone().cpu(), vc.clone().cpu()
    OP.store_kvcache(key.cpu(), value.cpu(), k_ref, v_ref, slots.cpu())
    k_gpu, v_gpu = kc.to(gpu), vc.to(gpu)
    pkg.kernels.store_kvcache(key.to(gpu), value.to(gpu), k_gpu, v_gpu, slots.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(k_gpu.cpu(), k_ref)
    assert torch.equal(v_gpu.cpu(), v_ref)


def test_store_config1_bit_exact(pkg, gpu):
    w = W.decode_one_layer(seed=0)
    _run_both(pkg, gpu, w["k_new"], w["v_new"], w["k_cache"], w["v_cache"], w["slot_mapping"])


def test_store_strided_value_view_of_qkv(pkg, gpu):
    # value is a strided view of the fused qkv output (row stride 4096), as in
    # Qwen3Attention.forward_decode (qwen3_naive.py:655).
    g = torch.Generator().manual_seed(1)
    n = 64
    qkv = torch.randn(n, 4096, generator=g).to(torch.bfloat16)
    k = qkv[:, 2048:3072].reshape(n, 8, 128).contiguous()
    v = qkv[:, 3072:].view(n, 8, 128)
    kc = torch.randn(8, 256, 8, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(8, 256, 8, 128, generator=g).to(torch.bfloat16)
    slots = torch.randperm(8 * 256, generator=g)[:n].to(torch.int32)
    print("[store] strided view", flush=True)
    k_ref, v_ref = kc.clone(), vc.clone()
    OP.store_kvcache(k, v, k_ref, v_ref, slots)
    qkv_g = qkv.to(gpu)
    kg, vg = kc.to(gpu), vc.to(gpu)
    pkg.kernels.store_kvcache(k.to(gpu), qkv_g[:, 3072:].view(n, 8, 128), kg, vg, slots.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)


def test_store_skips_minus_one_and_out_of_range(pkg, gpu):
    g = torch.Generator().manual_seed(2)
    key = torch.randn(5, 8, 128, generator=g).to(torch.bfloat16)
    val = torch.randn(5, 8, 128, generator=g).to(torch.bfloat16)
    kc = torch.zeros(2, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([3, -1, 511, 512, -7], dtype=torch.int32)  # 512 and -7 are out of range
    print("[store] -1 / out-of-range slots", flush=True)
    kg, vg = kc.to(gpu), vc.to(gpu)
    pkg.kernels.store_kvcache(key.to(gpu), val.to(gpu), kg, vg, slots.to(gpu))
    torch.cuda.synchronize()
    k_ref, v_ref = kc.clone(), vc.clone()
    OP.store_kvcache(key, val, k_ref, v_ref, torch.tensor([3, -1, 511, -1, -1]))
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)


def test_store_prefill_chunk_size(pkg, gpu):
    # 8192 new tokens (16 sequences x 512-token chunk) into a shuffled pool.
    g = torch.Generator().manual_seed(3)
    n, nb = 8192, 48
    key = torch.randn(n, 8, 128, generator=g).to(torch.bfloat16)
    val = torch.randn(n, 8, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, 256, 8, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, 256, 8, 128, generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * 256, generator=g)[:n].to(torch.int32)
    _run_both(pkg, gpu, key, val, kc, vc, slots)


def test_store_unaligned_rows_use_scalar_path(pkg, gpu):
    # Row stride 1025 elements is not a multiple of 8: the 2-byte path runs.
    g = torch.Generator().manual_seed(4)
    base = torch.randn(16, 1025, generator=g).to(torch.bfloat16)
    key = base[:, :1024].view(16, 8, 128)
    val = base[:, 1:].reshape(16, 8, 128)
    kc = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.arange(16, dtype=torch.int32) * 3
    print("[store] unaligned", flush=True)
    bg = base.to(gpu)
    kg, vg = kc.to(gpu), vc.to(gpu)
    pkg.kernels.store_kvcache(bg[:, :1024].view(16, 8, 128), bg[:, 1:].as_strided((16, 8, 128), (1025, 128, 1)),
                              kg, vg, slots.to(gpu))
    torch.cuda.synchronize()
    k_ref, v_ref = kc.clone(), vc.clone()
    OP.store_kvcache(key, base[:, 1:].as_strided((16, 8, 128), (1025, 128, 1)), k_ref, v_ref, slots)
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)


def test_store_empty_is_noop(pkg, gpu):
    kc = torch.ones(1, 256, 8, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.ones_like(kc)
    e = torch.empty(0, 8, 128, dtype=torch.bfloat16, device=gpu)
    pkg.kernels.store_kvcache(e, e, kc, vc, torch.empty(0, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    assert kc.sum().item() == 256 * 8 * 128


def test_store_rejects_bad_inputs(pkg, gpu):
    kc = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(2, 8, 128, dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError):
        pkg.kernels.store_kvcache(k, k, kc, kc, torch.zeros(2, dtype=torch.int32, device=gpu))
    kb = k.to(torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.kernels.store_kvcache(kb, kb, kc, kc, torch.zeros(3, dtype=torch.int32, device=gpu))
