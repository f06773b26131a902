"""Build-time checks of the compiled gfx950 code.

1. No ``v_mfma_scale`` may read an E8M0 scale operand from a register inside
   its own destination range.
2. No LDS DMA (``global_load_lds_*`` / ``buffer_load_* ... lds``) may directly
   follow an SALU write of M0: GFX9-family parts need one wait state between
   the two, and the compiler cannot insert it inside inline asm.
3. No instruction written as inline asm may read or write the destination of
   an MFMA within the 20 wait states that follow it (a 16-pass XDL MFMA on
   gfx950), nor write one of its SrcC registers within 15.  The hardware does
   not interlock these; the compiler inserts the wait states for its own
   instructions but does not look at the operands of inline asm.  This check
   reads the compiler's assembly output (``-save-temps``), where inline asm is
   bracketed by ``;;#ASMSTART`` / ``;;#ASMEND``.

When the accumulator input of a scaled MFMA is the constant 0, the compiler
does not tie the destination to it and can allocate the destination over a
scale register that dies at the instruction; the MFMA then reads a scale that
its own result has overwritten.  The kernels keep such scales live past the
MFMA; this check, run on every object ``build_lib.py`` produces, catches a
compiler allocation that slips through.

It disassembles only code built here: the device code object embedded in
the host object's ``.hip_fatbin`` section, extracted with the ROCm LLVM tools.
"""

from __future__ import annotations

import os
import re
import subprocess
import tempfile

LLVM_BIN = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
_VEC = re.compile(r"v\[(\d+):(\d+)\]")
_REG = re.compile(r"v(\d+)$")


def tools_available() -> bool:
    return all(os.path.exists(os.path.join(LLVM_BIN, t))
               for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))


def disassemble(obj: str) -> str:
    """Disassembly of the gfx950 code object inside a hipcc-built object."""
    with tempfile.TemporaryDirectory() as td:
        fat, co, junk = (os.path.join(td, n) for n in ("fat.bin", "dev.co", "junk.o"))
        subprocess.run([os.path.join(LLVM_BIN, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", obj, junk],
                       check=True, capture_output=True)
        subprocess.run([os.path.join(LLVM_BIN, "clang-offload-bundler"), "--type=o", f"--targets={TARGET}",
                        f"--input={fat}", f"--output={co}", "--unbundle"], check=True, capture_output=True)
        r = subprocess.run([os.path.join(LLVM_BIN, "llvm-objdump"), "-d", co], check=True, capture_output=True,
                           text=True)
        return r.stdout


def scale_dst_overlaps(asm: str) -> list:
    """Scaled-MFMA lines whose scale operand register lies in the destination range."""
    bad = []
    for line in asm.splitlines():
        t = line.strip()
        if not t.startswith("v_mfma_scale"):
            continue
        ops = [o.strip() for o in t.split("//")[0].split(None, 1)[1].split(",")]
        d = _VEC.match(ops[0])
        if not d:
            continue
        lo, hi = int(d.group(1)), int(d.group(2))
        for o in ops[4:6]:
            m = _REG.match(o.split()[0]) if o else None
            if m and lo <= int(m.group(1)) <= hi:
                bad.append(t.split("//")[0].strip())
                break
    return bad


def _instructions(asm: str) -> list:
    """Instruction mnemonics + operands in program order (labels and blanks dropped)."""
    out = []
    for line in asm.splitlines():
        t = line.split("//")[0].strip()
        if not t or t.endswith(":") or t.startswith(("Disassembly", ".")) or "file format" in t:
            continue
        out.append(t)
    return out


def _writes_m0(ins: str) -> bool:
    parts = ins.split(None, 1)
    return parts[0].startswith("s_") and len(parts) > 1 and parts[1].split(",")[0].strip() == "m0"


def _is_lds_dma(ins: str) -> bool:
    op = ins.split(None, 1)[0]
    return op.startswith("global_load_lds") or (op.startswith("buffer_load") and re.search(r"\blds\b", ins) is not None)


def m0_lds_dma_hazards(asm: str) -> list:
    """LDS DMA instructions issued directly after an SALU write of M0."""
    ins = _instructions(asm)
    return [f"{ins[i - 1]} ; {ins[i]}" for i in range(1, len(ins)) if _is_lds_dma(ins[i]) and _writes_m0(ins[i - 1])]


_REGS = re.compile(r"\b([vsa])(\d+)\b|\b([vsa])\[(\d+):(\d+)\]")
XDL_READ_WAIT = 20   # wait states before a VALU/VMEM/LDS access of a 16-pass XDL result (gfx950)
XDL_SRCC_WAR_WAIT = 15


def _reg_set(ops: str) -> set:
    out = set()
    for m in _REGS.finditer(ops):
        if m.group(1):
            out.add((m.group(1), int(m.group(2))))
        else:
            out.update((m.group(3), r) for r in range(int(m.group(4)), int(m.group(5)) + 1))
    return out


def _asm_listing(s_text: str) -> list:
    """(instruction, from_inline_asm) in program order from compiler assembly."""
    out, in_asm = [], False
    for line in s_text.splitlines():
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        t = t.split(";")[0].strip()
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        out.append((t, in_asm))
    return out


def asm_mfma_operand_hazards(s_text: str) -> list:
    """Inline-asm instructions that touch an MFMA's registers inside its hazard window."""
    ins = _asm_listing(s_text)
    bad = []
    for i, (t, _) in enumerate(ins):
        if not t.startswith("v_mfma"):
            continue
        ops = [o.strip() for o in t.split(None, 1)[1].split(",")]
        dst = _reg_set(ops[0])
        srcc = _reg_set(ops[3]) if len(ops) > 3 else set()
        ws = 0
        for t2, from_asm in ins[i + 1:]:
            if t2.startswith("s_nop"):
                ws += int(t2.split()[1]) + 1
                continue
            if t2.startswith(("s_branch", "s_setpc", "s_endpgm")):
                break
            ws += 1
            if ws > XDL_READ_WAIT:
                break
            if not from_asm or t2.startswith("v_mfma"):
                continue
            parts = t2.split(None, 1)
            if len(parts) < 2:
                continue
            regs = _reg_set(parts[1])
            d2 = _reg_set(parts[1].split(",")[0])
            if regs & dst or (ws <= XDL_SRCC_WAR_WAIT and d2 & srcc):
                bad.append(f"{t} ... {t2} ({ws} issue slots later)")
    return bad


def check_assembly(s_path: str) -> list:
    with open(s_path) as f:
        return asm_mfma_operand_hazards(f.read())


def check_object(obj: str) -> list:
    asm = disassemble(obj)
    return scale_dst_overlaps(asm) + m0_lds_dma_hazards(asm)


def scratch_kernels(s_text: str, name_part: str = "attn_fwd_kernel") -> list:
    """Kernels (whose symbol contains ``name_part``) that spill registers:
    [(symbol, scratch loads and stores in the body)] from a device assembly
    file.  (A reserved private segment that no instruction touches is not
    counted.)"""
    out = []
    for m in re.finditer(r"^(\S*" + re.escape(name_part) + r"\S*):[^\n]*\n(.*?)^\.Lfunc_end", s_text, re.M | re.S):
        n = len(re.findall(r"^\s*scratch_(?:load|store)\w*\s", m.group(2), re.M))
        if n:
            out.append((m.group(1), n))
    return out
