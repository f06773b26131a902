"""Checks of the built gfx950 code that need no GPU.

The scaled MFMAs of the attention and self-test kernels must not read an E8M0
scale from a register inside their own destination range (a compiler
allocation that makes the MFMA read a scale its result has overwritten; the
kernels keep those scales live past the MFMA).  Runs on the objects the last
build left in ``_build``; skipped when there is no build.
"""

import glob
import os
import sys

import pytest

HERE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "low-bit-attention-fake-quant_amd")
sys.path.insert(0, HERE)
import mfma_check  # noqa: E402

OBJS = sorted(glob.glob(os.path.join(HERE, "_build", "lbfq_*.o")))


def test_parser_flags_overlap():
    asm = ("\tv_mfma_scale_f32_32x32x64_f8f6f4 v[64:79], v[136:143], v[104:111], 0, v64, v166 op_sel_hi:[0,0,0]\n"
           "\tv_mfma_scale_f32_32x32x64_f8f6f4 v[0:15], v[16:23], v[24:31], v[0:15], v40, v41 op_sel_hi:[0,0,0]\n")
    bad = mfma_check.scale_dst_overlaps(asm)
    assert len(bad) == 1 and "v64, v166" in bad[0]


@pytest.mark.skipif(not OBJS or not mfma_check.tools_available(), reason="no build objects or ROCm LLVM tools")
@pytest.mark.parametrize("obj", OBJS, ids=[os.path.basename(o) for o in OBJS])
def test_no_scale_operand_in_mfma_destination(obj):
    assert mfma_check.check_object(obj) == []
