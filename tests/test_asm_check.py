"""The build-time check of hand-placed LDS waits (asm_check.py).

The prefill kernel's inline-asm LDS reads are waited for by hand-placed
``s_waitcnt lgkmcnt(N)``; the check follows the built device assembly and
fails the build if a scalar load is in flight across such a wait, or if an
LDS read's destination registers are touched before a wait retires it.
The planted cases below are small assembly texts, one mistake each, so a
checker that misses a rule fails here; the last test compiles the real
kernel and requires it clean (and the check not to be vacuous on it).
"""
from __future__ import annotations

import importlib.util
import re
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "qwen3-naive-inference_amd"


def _load(name: str, path: Path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


A = _load("qmi_asm_check", PKG_DIR / "asm_check.py")


def _kernel(body: str) -> str:
    lines = [ln.strip() for ln in body.strip().splitlines()]
    return "k: ; @k\n" + "\n".join("\t" + ln if not ln.endswith(":") else ln
                                    for ln in lines) + "\n.Lfunc_end0:\n"


def test_ordered_waits_pass():
    asm = _kernel("""
        ds_read_b128 v[0:3], v10
        ds_read_b64_tr_b16 v[4:5], v11 offset:64
        s_waitcnt lgkmcnt(1)
        v_mfma_f32_16x16x32_bf16 v[20:23], v[0:3], v[30:33], v[20:23]
        s_waitcnt lgkmcnt(0)
        v_mov_b32 v24, v4
        s_endpgm
    """)
    assert A.check_asm(asm) == []


def test_scalar_load_across_partial_wait_fails():
    asm = _kernel("""
        ds_read_b128 v[0:3], v10
        ds_read_b128 v[4:7], v10 offset:16
        s_load_dword s4, s[0:1], 0x0
        s_waitcnt lgkmcnt(1)
        v_mov_b32 v20, v0
        s_endpgm
    """)
    errs = A.check_asm(asm)
    assert any("scalar load in flight" in e for e in errs), errs


def test_scalar_load_waited_to_zero_passes():
    asm = _kernel("""
        s_load_dword s4, s[0:1], 0x0
        ds_read_b128 v[0:3], v10
        s_waitcnt lgkmcnt(0)
        v_mov_b32 v20, v0
        ds_read_b128 v[4:7], v10
        ds_read_b128 v[8:11], v10 offset:16
        s_waitcnt lgkmcnt(1)
        v_mov_b32 v21, v4
        s_endpgm
    """)
    assert A.check_asm(asm) == []


def test_destination_read_before_wait_fails():
    asm = _kernel("""
        ds_read_b128 v[0:3], v10
        v_mov_b32 v20, v1
        s_waitcnt lgkmcnt(0)
        s_endpgm
    """)
    errs = A.check_asm(asm)
    assert any("before the LDS read" in e for e in errs), errs


def test_count_too_weak_fails():
    # lgkmcnt(1) retires only the older read; the newer one is used early.
    asm = _kernel("""
        ds_read_b128 v[0:3], v10
        ds_read_b128 v[4:7], v10 offset:16
        s_waitcnt lgkmcnt(1)
        v_mov_b32 v20, v4
        s_endpgm
    """)
    assert A.check_asm(asm), "a use of the newest read after lgkmcnt(1) must fail"


def test_destination_overwritten_before_wait_fails():
    asm = _kernel("""
        ds_read_b128 v[0:3], v10
        v_mov_b32 v2, 0
        s_waitcnt lgkmcnt(0)
        s_endpgm
    """)
    assert A.check_asm(asm)


def test_loop_carried_read():
    ok = _kernel("""
        ds_read_b128 v[0:3], v10
        .LBB0_1:
        s_waitcnt lgkmcnt(0)
        v_mov_b32 v20, v0
        ds_read_b128 v[0:3], v10
        s_cbranch_scc1 .LBB0_1
        s_waitcnt lgkmcnt(0)
        s_endpgm
    """)
    assert A.check_asm(ok) == []
    # The read issued at the end of the body reaches the use at the top of
    # the next iteration through the back edge with no wait in between.
    bad = _kernel("""
        s_waitcnt lgkmcnt(0)
        .LBB0_1:
        v_mov_b32 v20, v0
        ds_read_b128 v[0:3], v10
        s_cbranch_scc1 .LBB0_1
        s_waitcnt lgkmcnt(0)
        s_endpgm
    """)
    assert A.check_asm(bad)


def test_read_pending_on_one_branch_only_fails():
    asm = _kernel("""
        s_cbranch_scc1 .LBB0_2
        ds_read_b128 v[0:3], v10
        .LBB0_2:
        v_mov_b32 v20, v0
        s_waitcnt lgkmcnt(0)
        s_endpgm
    """)
    assert A.check_asm(asm)


def test_m0_rules():
    ok = _kernel("""
        s_mov_b32 m0, s5
        s_nop 0
        global_load_lds_dwordx4 v1, s[2:3]
        s_endpgm
    """)
    assert A.check_asm(ok) == []
    other_writer = _kernel("""
        s_mov_b32 m0, -1
        ds_read_b32 v0, v1
        s_waitcnt lgkmcnt(0)
        s_endpgm
    """)
    assert A.check_asm(other_writer)
    reader = _kernel("""
        s_mov_b32 s6, m0
        s_endpgm
    """)
    assert A.check_asm(reader)


def test_prefill_kernel_assembly_is_clean():
    b = _load("qmi_build", PKG_DIR / "build.py")
    src = PKG_DIR / "csrc" / "varlen_prefill.hip"
    flags = [*b.HIPCC_FLAGS, *b.EXTRA_FLAGS.get(src.name, [])]
    try:
        asm = A.device_asm(src, b.hipcc_path(), flags)
    except (RuntimeError, FileNotFoundError) as exc:  # no hipcc on this host
        pytest.skip(f"hipcc unavailable: {exc}")
    kernels = [k for k in A._functions(asm) if "varlen_prefill_kernel" in k]
    assert len(kernels) == 6, kernels           # GQA ratios 1, 2, 4 x grid / queue mode
    # Not vacuous: the kernels hold the inline-asm reads, partial waits and
    # direct loads the check is about.
    assert len(re.findall(r"ds_read_b128 ", asm)) >= 6 * 32
    assert len(re.findall(r"ds_read_b64_tr_b16 ", asm)) >= 6 * 32
    assert len(re.findall(r"lgkmcnt\([1-9]\d*\)", asm)) >= 6 * 8
    assert len(re.findall(r"global_load_lds_dwordx4 ", asm)) >= 6 * 8
    assert A.check_asm(asm) == []
