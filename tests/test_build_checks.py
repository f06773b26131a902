"""Checks of the built gfx950 code that need no GPU.

The scaled MFMAs of the attention and self-test kernels must not read an E8M0
scale from a register inside their own destination range (a compiler
allocation that makes the MFMA read a scale its result has overwritten; the
kernels keep those scales live past the MFMA).  No LDS DMA may directly
follow an SALU write of M0 (GFX9-family parts need one wait state between
them; inline asm hides the pair from the compiler's hazard recognizer).  No
inline asm may touch an MFMA's destination or SrcC registers inside the
hazard window (gfx950 does not interlock XDL results; the compiler only
protects its own instructions).  No attention kernel spills registers to
scratch memory.  Runs on the objects the last build left in ``_build``; skipped when there is no
build.
"""

import glob
import os
import sys

import pytest

HERE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "low-bit-attention-fake-quant_amd")
sys.path.insert(0, HERE)
import mfma_check  # noqa: E402

# the units' objects (not the device / host temporaries of -save-temps)
OBJS = sorted(o for o in glob.glob(os.path.join(HERE, "_build", "lbfq_*.o")) if "-hip-" not in o and "-host-" not in o)


def test_parser_flags_overlap():
    asm = ("\tv_mfma_scale_f32_32x32x64_f8f6f4 v[64:79], v[136:143], v[104:111], 0, v64, v166 op_sel_hi:[0,0,0]\n"
           "\tv_mfma_scale_f32_32x32x64_f8f6f4 v[0:15], v[16:23], v[24:31], v[0:15], v40, v41 op_sel_hi:[0,0,0]\n")
    bad = mfma_check.scale_dst_overlaps(asm)
    assert len(bad) == 1 and "v64, v166" in bad[0]


def test_parser_flags_m0_then_lds_dma():
    asm = ("kernel:\n"
           "\ts_mov_b32 m0, s87                     // 000000001000: BEFC0057\n"
           "\tglobal_load_lds_dwordx4 v186, s[8:9]  // 000000001004: DDF48000 00087DBA\n"
           "\ts_mov_b32 m0, s23\n"
           "\ts_nop 0\n"
           "\tglobal_load_lds_dword v184, s[2:3]\n"
           "\ts_mov_b32 m0, s6\n"
           "\tbuffer_load_dword v1, s[4:7], 0 offen lds\n"
           "\ts_mov_b32 s6, m0\n"
           "\tglobal_load_lds_dword v184, s[2:3]\n")
    bad = mfma_check.m0_lds_dma_hazards(asm)
    assert len(bad) == 2
    assert bad[0].startswith("s_mov_b32 m0, s87") and bad[1].startswith("s_mov_b32 m0, s6 ;")


def test_parser_flags_inline_asm_reading_mfma_result():
    mfma = "\tv_mfma_scale_f32_32x32x64_f8f6f4 v[80:95], v[136:143], v[104:111], 0, v114, v182 op_sel_hi:[0,0,0]\n"
    asm_read = "\t;;#ASMSTART\n\tv_max3_f32 v139, v86, v87, v88\n\t;;#ASMEND\n"
    compiler_read = "\tv_max3_f32 v139, v86, v87, v88\n"
    filler = "\tv_add_f32_e32 v1, v2, v3\n"
    # inline asm 6 slots after the MFMA: flagged; after 15 + 4 + 1 nop wait states: clean
    assert len(mfma_check.asm_mfma_operand_hazards(mfma + filler * 5 + asm_read)) == 1
    assert mfma_check.asm_mfma_operand_hazards(mfma + "\ts_nop 15\n\ts_nop 3\n" + filler + asm_read) == []
    # the same read by the compiler is its own business (it inserts the wait states)
    assert mfma_check.asm_mfma_operand_hazards(mfma + compiler_read) == []
    # inline asm writing a SrcC register of an in-flight MFMA
    acc = "\tv_mfma_scale_f32_32x32x64_f8f6f4 v[0:15], v[16:23], v[24:31], v[40:55], v60, v61 op_sel_hi:[0,0,0]\n"
    war = "\t;;#ASMSTART\n\tv_mov_b32 v41, 0\n\t;;#ASMEND\n"
    assert len(mfma_check.asm_mfma_operand_hazards(acc + war)) == 1


@pytest.mark.skipif(not OBJS or not mfma_check.tools_available(), reason="no build objects or ROCm LLVM tools")
@pytest.mark.parametrize("obj", OBJS, ids=[os.path.basename(o) for o in OBJS])
def test_no_scale_operand_in_mfma_destination_and_no_m0_dma_hazard(obj):
    assert mfma_check.check_object(obj) == []


@pytest.mark.parametrize("obj", OBJS, ids=[os.path.basename(o) for o in OBJS])
def test_no_inline_asm_inside_mfma_hazard_window(obj):
    import build_lib
    s_path = build_lib.device_asm(obj)
    if not os.path.exists(s_path):
        pytest.skip("no device assembly (built without -save-temps)")
    assert mfma_check.check_assembly(s_path) == []


def test_parser_finds_scratch_kernels():
    text = ("_ZN9lbfq_attn15attn_fwd_kernelILi128EEEvNS_5KArgsE: ; @x\n"
            "\tv_mov_b32 v0, 0\n\tscratch_store_dword off, v2, off offset:28 ; 4-byte Folded Spill\n"
            "\tscratch_load_dword v2, off, off offset:28 ; 4-byte Folded Reload\n.Lfunc_end0:\n"
            "_ZN9lbfq_attn15attn_fwd_kernelILi64EEEvNS_5KArgsE:\n\tv_mov_b32 v0, 0\n.Lfunc_end1:\n"
            "_ZN4lbfq11other_kernelEv:\n\tscratch_store_dword off, v2, off\n.Lfunc_end2:\n")
    assert mfma_check.scratch_kernels(text) == [("_ZN9lbfq_attn15attn_fwd_kernelILi128EEEvNS_5KArgsE", 2)]


ATTN_OBJS = [o for o in OBJS if os.path.basename(o).startswith("lbfq_attn")]


@pytest.mark.parametrize("obj", ATTN_OBJS, ids=[os.path.basename(o) for o in ATTN_OBJS])
def test_attention_kernels_do_not_spill(obj):
    import build_lib
    s_path = build_lib.device_asm(obj)
    if not os.path.exists(s_path):
        pytest.skip("no device assembly (built without -save-temps)")
    with open(s_path) as f:
        assert mfma_check.scratch_kernels(f.read()) == []

