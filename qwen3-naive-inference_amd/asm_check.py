"""Static check of hand-placed LDS waits in the built gfx950 assembly.

The prefill kernel issues its LDS operand reads (``ds_read_b128``,
``ds_read_b64_tr_b16``) as inline asm and waits for them with hand-placed
``s_waitcnt lgkmcnt(N)``.  The compiler does not know that the asm outputs
arrive late, so two things it may do would read stale LDS data without any
error:

* put a scalar memory load (``s_load_*``; also counted by lgkmcnt, and
  returning out of order with the LDS reads) in flight across a
  ``lgkmcnt(N)`` wait with N > 0, so that the count no longer says which LDS
  reads have landed;
* read, copy or overwrite the destination registers of an LDS read before a
  wait has retired it (a register-allocator copy, a spill).

This module compiles a source to device assembly and follows every
instruction of every kernel along the control-flow graph, keeping the queue
of outstanding LDS/scalar-memory operations: LDS operations retire in issue
order, so ``lgkmcnt(N)`` retires all but the newest N of them, but only when
no scalar load is outstanding.  It also checks that M0, which the inline-asm
direct global->LDS loads set, is written only by those loads' own
``s_mov_b32 m0`` and read only by the loads that directly follow it.

The check applies to every LDS read of the kernel, the compiler's own
included (those carry correct compiler-placed waits, so they pass too).
``build.py`` runs it on every build; a violation fails the build.
"""
from __future__ import annotations

import re
import subprocess
from dataclasses import dataclass, field
from pathlib import Path

_REG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")
_LABEL = re.compile(r"^(\.?[A-Za-z_$][\w.$]*):")


class AsmCheckError(RuntimeError):
    pass


def _regs(text: str) -> set[tuple[str, int]]:
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.add((m.group(1), int(m.group(2))))
        else:
            lo, hi = int(m.group(4)), int(m.group(5))
            out.update((m.group(3), r) for r in range(lo, hi + 1))
    return out


@dataclass
class _Insn:
    line: int
    op: str
    args: str


@dataclass
class _Block:
    name: str
    insns: list[_Insn] = field(default_factory=list)
    succ: list[str] = field(default_factory=list)


# The LDS counter (lgkmcnt) is 4 bits: a wave holds at most 15 LDS
# operations in flight, so only the newest 15 of a longer sequence can
# still be pending.
_MAX_PENDING = 15


@dataclass(frozen=True)
class _State:
    """Outstanding LGKM operations at a program point.

    ``lds``: one entry per LDS operation in flight, oldest first, each the
    destination registers it will write and the lines that issued it.
    ``smem``: lines of scalar loads possibly in flight (they retire out of
    order, so only lgkmcnt(0) is known to retire them)."""
    lds: tuple = ()
    smem: frozenset = frozenset()

    def join(self, other: "_State") -> "_State":
        # Entries are aligned at the newest end (waits retire from the
        # oldest), each position keeping the union of both paths.
        a, b = self.lds, other.lds
        n = max(len(a), len(b))
        a = ((frozenset(), frozenset()),) * (n - len(a)) + a
        b = ((frozenset(), frozenset()),) * (n - len(b)) + b
        lds = tuple((x[0] | y[0], x[1] | y[1]) for x, y in zip(a, b))
        return _State(lds, self.smem | other.smem)


def _functions(asm: str) -> dict[str, list[tuple[int, str]]]:
    """Kernel name -> (line number, text) of its body, up to .Lfunc_end."""
    funcs: dict[str, list[tuple[int, str]]] = {}
    cur = None
    for no, raw in enumerate(asm.splitlines(), 1):
        line = raw.split(";", 1)[0].rstrip()
        m = _LABEL.match(line.strip())
        if m and not m.group(1).startswith("."):
            # A function's label carries the assembler's "; @name" comment.
            if "; @" in raw:
                cur = m.group(1)
                funcs[cur] = []
            else:
                cur = None
            continue
        if cur is None:
            continue
        if line.strip().startswith(".Lfunc_end"):
            cur = None
            continue
        funcs[cur].append((no, line))
    return funcs


def _blocks(body: list[tuple[int, str]]) -> tuple[list[_Block], dict[str, _Block]]:
    blocks: list[_Block] = [_Block("<entry>")]
    for no, line in body:
        s = line.strip()
        if not s:
            continue
        m = _LABEL.match(s)
        if m:
            blocks.append(_Block(m.group(1)))
            continue
        if s.startswith("."):
            continue                 # directive
        op, _, args = s.partition(" ")
        blocks[-1].insns.append(_Insn(no, op, args.strip()))
        if op.startswith("s_cbranch") or op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            blocks.append(_Block(f"<after {no}>"))
    by_name = {b.name: b for b in blocks}
    for i, b in enumerate(blocks):
        last = b.insns[-1] if b.insns else None
        if last is not None and (last.op.startswith("s_cbranch") or last.op == "s_branch"):
            tgt = last.args.split()[0]
            if tgt not in by_name:
                raise AsmCheckError(f"branch to unknown label {tgt} (line {last.line})")
            b.succ.append(tgt)
        if last is not None and last.op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            continue
        if i + 1 < len(blocks):
            b.succ.append(blocks[i + 1].name)
    return blocks, by_name


def _step(kernel: str, insn: _Insn, st: _State, errors: list[str]) -> _State:
    op = insn.op
    lds, smem = list(st.lds), st.smem
    if op == "s_waitcnt":
        m = _LGKM.search(insn.args)
        if m:
            n = int(m.group(1))
            if n == 0:
                lds, smem = [], frozenset()
            elif smem:
                errors.append(f"{kernel}: line {insn.line}: lgkmcnt({n}) with a scalar load in "
                              f"flight (issued at line(s) {sorted(smem)}); LDS reads may not "
                              f"have landed")
            else:
                del lds[: max(0, len(lds) - n)]
        return _State(tuple(lds), smem)
    regs = _regs(insn.args)
    for dests, lines in lds:
        if dests & regs:
            errors.append(f"{kernel}: line {insn.line}: `{op} {insn.args}` touches "
                          f"{sorted(dests & regs)[:4]} before the LDS read of line(s) "
                          f"{sorted(lines)} is waited for")
    if op.startswith("s_load") or op.startswith("s_buffer_load") or op in (
            "s_memtime", "s_memrealtime", "s_sendmsg", "s_sendmsghalt", "s_dcache_inv"):
        smem = smem | {insn.line}
    elif op.startswith("ds_"):
        dst = frozenset()
        if "read" in op or op.startswith(("ds_bpermute", "ds_permute", "ds_swizzle")) \
                or "_rtn" in op:
            dst = frozenset(_regs(insn.args.split(",")[0]))
        lds.append((dst, frozenset({insn.line})))
        del lds[: max(0, len(lds) - _MAX_PENDING)]
    return _State(tuple(lds), smem)


def _check_m0(kernel: str, blocks: list[_Block], errors: list[str]) -> None:
    for b in blocks:
        for i, insn in enumerate(b.insns):
            args = insn.args
            if re.search(r"\bm0\b", args) is None:
                continue
            dst = args.split(",")[0].strip()
            if insn.op == "s_mov_b32" and dst == "m0":
                nxt = b.insns[i + 1: i + 3]
                ops = [n.op for n in nxt]
                if ops[:2] != ["s_nop", "global_load_lds_dwordx4"]:
                    errors.append(f"{kernel}: line {insn.line}: M0 written by something other "
                                  f"than a direct global->LDS load sequence ({ops})")
            else:
                errors.append(f"{kernel}: line {insn.line}: `{insn.op} {args}` uses M0")


def check_asm(asm: str, kernel_filter: str = "") -> list[str]:
    """Return the list of violations in an assembly text (empty = clean)."""
    errors: list[str] = []
    for kernel, body in _functions(asm).items():
        if kernel_filter not in kernel:
            continue
        blocks, by_name = _blocks(body)
        preds: dict[str, list[str]] = {b.name: [] for b in blocks}
        for b in blocks:
            for s in b.succ:
                preds[s].append(b.name)
        state_out: dict[str, _State] = {}
        work = [blocks[0].name]
        seen_err: set[str] = set()
        while work:
            name = work.pop()
            st = _State()
            for p in preds[name]:
                if p in state_out:
                    st = st.join(state_out[p])
            local: list[str] = []
            for insn in by_name[name].insns:
                st = _step(kernel, insn, st, local)
            for e in local:
                if e not in seen_err:
                    seen_err.add(e)
                    errors.append(e)
            if state_out.get(name) != st:
                state_out[name] = st
                work.extend(by_name[name].succ)
        _check_m0(kernel, blocks, errors)
    return errors


def device_asm(src: Path, hipcc: str, flags: list[str]) -> str:
    """Compile ``src`` to gfx950 device assembly and return the text."""
    tmp_dir = Path(__file__).resolve().parent / "_build"
    tmp_dir.mkdir(exist_ok=True)
    out = tmp_dir / (src.stem + ".device.s")
    cmd = [hipcc, *flags, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise AsmCheckError(f"device assembly of {src.name} failed:\n{res.stderr}")
    return out.read_text()


def check_source(src: Path, hipcc: str, flags: list[str], kernel_filter: str = "") -> None:
    errors = check_asm(device_asm(src, hipcc, flags), kernel_filter)
    if errors:
        raise AsmCheckError(f"{src.name}: hand-placed LDS waits are unsafe in the built code:\n"
                            + "\n".join(errors[:20]))
