"""Build-time check of the compiled gfx950 code: no ``v_mfma_scale`` may read
an E8M0 scale operand from a register inside its own destination range.

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


def check_object(obj: str) -> list:
    return scale_dst_overlaps(disassemble(obj))
