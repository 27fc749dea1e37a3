"""Build the gfx950 shared library ``libqwen3mi.so`` from ``csrc/*.hip``.

The library is a plain C-ABI ``.so`` (no torch types in any signature) built
in-tree with ``hipcc`` so it travels with the source tree.  Each ``.hip``
file is compiled to an object in parallel and then linked once.

Usage: ``python -m`` is not possible for this package directory name, so run
``python qwen3-naive-inference_amd/build.py`` or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures
import importlib.util
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libqwen3mi.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from emitting packed-fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]

# Per-file additions.  The prefill kernel's score maxima are fmaxf chains over
# MFMA results; with NaN-quieting semantics the compiler puts a canonicalising
# v_max_f32 x, x, x in front of every operand, with relaxed NaN handling the
# chains become v_max3_f32.  That kernel never produces a NaN score from
# finite inputs (stale page rows are masked to -inf before any maximum).
#
# The prefill kernel takes its next work-queue ticket with one atomic by one
# thread and uses the value only after the next item's loads; the AMDGPU
# atomic optimizer would rewrite that atomic into a wave-wide form whose
# result is consumed (and waited for) at once.
EXTRA_FLAGS = {
    "varlen_prefill.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}

# Sources whose kernels place LDS waits by hand (inline-asm LDS reads with
# explicit lgkmcnt waits, inline-asm direct global->LDS loads through M0).
# Their device assembly is checked on every build (asm_check.py).
ASM_CHECKED = ("varlen_prefill.hip", "linear_rows.hip", "lm_head.hip")


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc_path(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    for line in (res.stdout + res.stderr).splitlines():
        if line.strip() and noise not in line and verbose:
            print(line)
    return obj


def _load_asm_check():
    spec = importlib.util.spec_from_file_location("qmi_asm_check", PKG_DIR / "asm_check.py")
    mod = sys.modules.get(spec.name)
    if mod is None:
        mod = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = mod
        spec.loader.exec_module(mod)
    return mod


def _asm_check(mod, src: Path) -> None:
    mod.check_source(src, hipcc_path(), [*HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, [])])


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libqwen3mi.so``.

    Always recompiles (this is the build check) and checks the hand-placed
    LDS waits of the ``ASM_CHECKED`` sources in their device assembly;
    returns the library path.
    """
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)), 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        mod = _load_asm_check()
        checks = [ex.submit(_asm_check, mod, s) for s in srcs if s.name in ASM_CHECKED]
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
        for c in checks:
            c.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc_path(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
