"""Compile liblbfq_hip.so (all HIP kernels + the C ABI) for gfx950.

Each ``csrc/*.hip`` translation unit is compiled with hipcc into an object,
then linked into ``low_bit_fake_quant/liblbfq_hip.so`` (in-tree, next to the
Python package that loads it).  The prepass / k-means translation units are
compiled with ``-ffp-contract=off`` so their arithmetic is exactly the
documented op sequence (the CPU oracle reproduces it bit for bit); the
attention units allow contraction and are built with -fno-honor-nans.  Packed-FP32 instructions are disabled
for all device code.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "low_bit_fake_quant", "liblbfq_hip.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("LBFQ_ARCH", "gfx950")

COMMON = [
    "hipcc", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# The attention units: no NaN ever flows through their arithmetic (scores are
# finite or -inf; the one 0/0 of BLASST's all-skipped zero-fill rows is formed
# in the epilogue and only converted to the output dtype by hardware), so
# fmaxf lowers to plain v_max / v_max3 without canonicalising its inputs.
ATTN_FLAGS = ["-fno-honor-nans"]
UNITS = {
    "lbfq_prepass.hip": ["-ffp-contract=off"],
    "lbfq_kmeans.hip": ["-ffp-contract=off"],
    "lbfq_qmk.hip": ["-ffp-contract=off"],
    "lbfq_probe.hip": ["-ffp-contract=off"],
    "lbfq_blasst_sim.hip": ["-ffp-contract=off"],
    "lbfq_attn.hip": ATTN_FLAGS,
    "lbfq_attn_p0.hip": ATTN_FLAGS,
    "lbfq_attn_p1.hip": ATTN_FLAGS,
    "lbfq_attn_p2.hip": ATTN_FLAGS,
    "lbfq_attn_b128_p0.hip": ATTN_FLAGS,
    "lbfq_attn_b128_p1.hip": ATTN_FLAGS,
    "lbfq_attn_b128_p2.hip": ATTN_FLAGS,
    "lbfq_sdpa.hip": ["-ffp-contract=off"],
}


def _compile(unit: str, extra: list[str]) -> str:
    src = os.path.join(CSRC, unit)
    obj = os.path.join(BUILD, unit.replace(".hip", ".o"))
    # -save-temps (run inside _build) keeps the device assembly, which the
    # inline-asm hazard check reads
    cmd = COMMON + extra + ["-save-temps", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True, cwd=BUILD)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {unit}:\n{' '.join(cmd)}\n{r.stderr}")
    return obj


def _check_mfma(objs: list[str]) -> None:
    sys.path.insert(0, HERE)
    import mfma_check
    if not mfma_check.tools_available():
        print("mfma_check: ROCm LLVM tools not found; code checks skipped", file=sys.stderr)
        return
    bad = {}
    for o in objs:
        found = mfma_check.check_object(o)
        s_path = device_asm(o)
        if os.path.exists(s_path):
            found += mfma_check.check_assembly(s_path)
        else:
            found.append(f"device assembly {os.path.basename(s_path)} missing (inline-asm hazard check not run)")
        if found:
            bad[o] = found
    for o in objs:  # spills of the attention kernels (a performance defect, reported)
        s_path = device_asm(o)
        if os.path.exists(s_path):
            with open(s_path) as f:
                for sym, nb in mfma_check.scratch_kernels(f.read()):
                    print(f"warning: {sym} spills registers ({nb} scratch loads / stores)", file=sys.stderr)
    if bad:
        lines = "\n".join(f"{os.path.basename(o)}: {x}" for o, b in bad.items() for x in b[:4])
        raise RuntimeError("gfx950 code check failed (a scaled MFMA reading a scale from its own destination "
                           "registers, an LDS DMA directly after an M0 write, or inline asm touching an MFMA's "
                           "registers inside its hazard window):\n" + lines)


def device_asm(obj: str) -> str:
    """Device assembly that -save-temps left next to a unit's object."""
    base = os.path.basename(obj)[:-2]
    return os.path.join(os.path.dirname(obj), f"{base}-hip-amdgcn-amd-amdhsa-{ARCH}.s")


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(UNITS), os.cpu_count() or 8)) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), UNITS.items()))
    _check_mfma(objs)
    tmp = OUT + ".tmp"
    cmd = ["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    build()
