"""The C-ABI library loads and exports every entry point include/qwen3mi.h declares
(CPU: no kernel is launched here, only argument validation that returns
before any HIP call)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qwen3mi.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"\b(qmi_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "qmi_store_kvcache" in names and "qmi_paged_decode_attention" in names
    assert "qmi_grpo_fused_loss" in names


def test_library_exports_every_declared_symbol(pkg):
    handle = ctypes.CDLL(str(pkg._lib.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(handle, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_table_covers_header(pkg):
    assert set(declared_functions()) == set(pkg._lib.SIGNATURES)


def test_error_strings_and_version(pkg):
    L = pkg._lib.lib()
    assert L.qmi_version() >= 100
    assert L.qmi_error_string(0) == b"success"
    assert b"NULL" in L.qmi_error_string(-1)
    assert b"workspace" in L.qmi_error_string(-5)


def test_validation_rejects_before_launch(pkg):
    L = pkg._lib.lib()
    # n_tokens == 0 is a no-op; negative sizes / NULL pointers are rejected.
    assert L.qmi_store_kvcache(None, 1024, None, 1024, None, None, None, 0, 1024, 16, None) == 0
    assert L.qmi_store_kvcache(None, 1024, None, 1024, None, None, None, 4, 1024, 16, None) == -1
    assert L.qmi_store_kvcache(None, 1024, None, 1024, None, None, None, -1, 1024, 16, None) == -2
    # unsupported head_dim / block size
    fake = 256
    st = L.qmi_paged_decode_attention(fake, 2048, 128, fake, fake, 16, 128, 16, 8, 128, fake, 1,
                                      fake, 4, 4, 4, 0.1, fake, 2048, 128, None, 0, 0, None)
    assert st == -4
    # GQA ratio 3 is rejected
    st = L.qmi_paged_decode_attention(fake, 2048, 128, fake, fake, 16, 256, 12, 4, 128, fake, 1,
                                      fake, 4, 4, 4, 0.1, fake, 2048, 128, None, 0, 0, None)
    assert st == -4
    # workspace required when a sequence can need more than one split
    need = L.qmi_paged_decode_workspace_bytes(4, 8, 16, 4, 1)
    assert need == 4 * 16 * 4 * 132 * 4
    st = L.qmi_paged_decode_attention(fake, 2048, 128, fake, fake, 16, 256, 16, 8, 128, fake, 1,
                                      fake, 4, 4, 4, 0.1, fake, 2048, 128, None, 0, 1, None)
    assert st == -5
    # the no-allocation variant validates the same way before any HIP call
    assert L.qmi_paged_decode_attention_noalloc(fake, 2048, 128, fake, fake, 16, 256, 16, 8, 128,
                                                fake, 1, fake, 4, 4, 0, 0.1, fake, 2048, 128, 0,
                                                None) == 0
    assert L.qmi_paged_decode_attention_noalloc(None, 2048, 128, fake, fake, 16, 256, 16, 8, 128,
                                                fake, 1, fake, 4, 4, 4, 0.1, fake, 2048, 128, 0,
                                                None) == -1
    assert L.qmi_paged_decode_attention_noalloc(fake, 2048, 128, fake, fake, 16, 128, 16, 8, 128,
                                                fake, 1, fake, 4, 4, 4, 0.1, fake, 2048, 128, 0,
                                                None) == -4
    assert b"scratch" in L.qmi_error_string(-6)
    assert 0 < L.qmi_grpo_fused_workspace_bytes(32, 512) < 4096
    assert L.qmi_ppo_clipped_loss(None, None, None, None, 1, 0, 2, 3, 0.2, 0, None, None, None) == -1
    assert L.qmi_ppo_clipped_loss(fake, fake, fake, fake, 1, 0, 2, 3, 0.2, 7, fake, None, None) == -4
    # fused lm_head: zero rows is a no-op; k above 64, hidden not a multiple of
    # 64, a non-positive temperature, a short workspace and a row count whose
    # item kernel would overflow its 32-bit item / step counts are rejected
    ws = L.qmi_lm_head_workspace_bytes(4, 151936, 0)
    assert ws >= 4 * (151936 // 32) * 8

    def sample(n_rows, hidden=1024, temp=1.0, top_k=0, ws_bytes=ws):
        return L.qmi_lm_head_sample(fake, 1024, n_rows, fake, 1024, 151936, hidden, temp, top_k,
                                    0, 0, None, fake, None, fake, ws_bytes, None)

    assert sample(0) == 0
    assert sample(4, top_k=65) == -4
    assert sample(4, hidden=1000) == -4
    assert sample(4, temp=0.0) == -2
    assert sample(4, ws_bytes=ws - 8) == -5
    assert sample(8_000_000, ws_bytes=1 << 62) == -4
    assert sample(7_000_000, ws_bytes=1 << 62, temp=0.0) == -2  # within the item-count limit
    assert L.qmi_lm_head_logprob(fake, 1024, 8_000_000, fake, 1024, 151936, 1024, fake, 1, fake,
                                 None, fake, 1 << 62, None) == -4
    assert L.qmi_lm_head_logprob(fake, 1024, 4, fake, 1024, 151936, 1024, None, 1, fake,
                                 None, fake, ws, None) == -1


def test_product_fails_loudly_without_library(pkg, monkeypatch, tmp_path):
    monkeypatch.setattr(pkg._lib, "_LIB", None)
    monkeypatch.setattr(pkg._lib, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(pkg._lib.QmiError):
        pkg._lib.lib()
