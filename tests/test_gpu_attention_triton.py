"""Kernel-level entry fake_quant_attention_triton (attention_triton.py:410-611)
as the reference's block study calls it (bench/eval_blasst_quant.py:151-209):
Q/K/V fp8_block-quantised with one block size, Q/K dequantised to bf16, V in
raw FP8 value units with its block scales applied in the K loop, elementwise
P, block_m = block_n = block size, the diagonal row-max start and BLASST.

Checked against the oracle's restatement of that kernel (oracle.attention):
the re-quantisation of the dequantised Q/K recovers the original codes
exactly; the output meets the north-star tolerance against the reference
algorithm replayed on the kernel's own scores; BLASST statistics equal the
replay's exactly; dense, cosine >= 0.9999 against the reference algorithm on
the exact (fp32) dequantised Q/K, with the gap to its bf16-rounded scores
(attention_triton.py dots of bf16 Q/K) printed: on these unsmoothed inputs with
outlier K channels that rounding alone moves the reference by ~1e-4 in cosine.
"""

import math

import pytest
import torch

import parity
from conftest import cosine
from oracle import attention as oattn

pytestmark = pytest.mark.gpu


def _study_inputs(block, n=1024, h=2, d=128, seed=31):
    from low_bit_fake_quant import fp8_block_dequant, fp8_block_quant
    from low_bit_fake_quant.wan import Workload, make_inputs
    q, k, v = make_inputs(Workload("t", h, n, d, None, field_grid=(4, 16, 16)), seed=seed)
    dev = torch.device("cuda:0")
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    qf, qs = fp8_block_quant(q, block_s=block)
    kf, ks = fp8_block_quant(k, block_s=block)
    vf, vs = fp8_block_quant(v, block_s=block)
    q_deq = fp8_block_dequant(qf, qs, block_s=block, dtype=torch.bfloat16)
    k_deq = fp8_block_dequant(kf, ks, block_s=block, dtype=torch.bfloat16)
    perm = (0, 2, 1, 3)
    q_bhsd = q_deq.permute(*perm).contiguous()
    k_bhsd = k_deq.permute(*perm).contiguous()
    v_bhsd = vf.to(torch.bfloat16).permute(*perm).contiguous()
    v_scale_bhd = torch.ones((1, h, d), dtype=torch.float32, device=dev)
    sm = 1.0 / math.sqrt(d)
    init = (q_bhsd.float() * k_bhsd.float()).sum(-1) * sm   # diagonal_rowmax_init
    q32 = fp8_block_dequant(qf, qs, block_s=block, dtype=torch.float32).permute(*perm).contiguous()
    k32 = fp8_block_dequant(kf, ks, block_s=block, dtype=torch.float32).permute(*perm).contiguous()
    return dict(q=q_bhsd, k=k_bhsd, v=v_bhsd, v_scale=v_scale_bhd, v_block_scale=vs.float().contiguous(),
                init=init, sm=sm, codes=(qf, kf), q32=q32, k32=k32)


@pytest.mark.parametrize("block", [64, 128])
@pytest.mark.parametrize("fill", [None, "mean_a1.5", "uta16_a1.5"])
def test_block_study_matches_oracle(gpu, block, fill):
    from low_bit_fake_quant.attention_kernel import attention_scores
    from low_bit_fake_quant.attention_triton import _requant_qk, fake_quant_attention_triton, triton_operands
    x = _study_inputs(block)
    kw = dict(sm_scale=x["sm"], p_max_offset=8, block_m=block, block_n=block, v_block_scale_bsh=x["v_block_scale"],
              v_block_size=block, p_quant_mode="elementwise", rowmax_init_bhs=x["init"])
    if fill is not None:
        kw.update(blasst_lambda=0.05, blasst_fill_mode=fill)
    out, stats = fake_quant_attention_triton(x["q"], x["k"], x["v"], x["v_scale"], return_blasst_stats=True, **kw)
    # the dequantised Q/K come back as the same codes, in blocks of the study's size
    for t, c in ((x["q"], x["codes"][0]), (x["k"], x["codes"][1])):
        codes, _, blk, exact = _requant_qk(t, block, t.shape[2])
        assert exact and blk == block
        assert torch.equal(codes, c.view(torch.uint8).permute(0, 2, 1, 3))
    ops, cfg, init = triton_operands(x["q"], x["k"], x["v"], x["v_scale"], **kw)
    u = attention_scores(ops, cfg, x["sm"]).reshape(ops.b, ops.h, ops.s, ops.s).cpu()
    okw = dict(sm_scale=x["sm"], p_max_offset=8, block_m=block, block_n=block, v_block_scale=x["v_block_scale"].cpu(),
               v_block_size=block, p_quant_mode="elementwise", rowmax_init=x["init"].cpu(),
               blasst_lambda=kw.get("blasst_lambda"), blasst_fill_mode=fill or "zero", return_blasst_stats=True)
    args = (x["q"].cpu(), x["k"].cpu(), x["v"].cpu(), x["v_scale"].cpu())
    rep, rstats, dbg = oattn.attention(*args, scores_log2=u, return_debug=True, **okw)
    parity.strict_check(out.cpu(), rep, f"study{block}-{fill}", allowance=dbg["flip_allowance"])
    if fill is not None:
        assert torch.equal(stats.cpu(), rstats)
        assert stats[..., 0].sum() > 0, "test input should make BLASST skip"
    else:
        ref, _ = oattn.attention(*args, **okw)
        ref32, _ = oattn.attention(x["q32"].cpu(), x["k32"].cpu(), *args[2:], **okw)
        c32, c16 = cosine(out.cpu(), ref32), cosine(out.cpu(), ref)
        print(f"study{block}: cosine vs reference on exact dequant {c32:.7f}, on bf16 dequant {c16:.7f} "
              f"(reference bf16 vs exact: {cosine(ref, ref32):.7f})")
        assert c32 >= parity.COS_MIN


def test_values_that_were_never_fp8(gpu):
    """Random bf16 Q/K (as the reference's own kernel test feeds it): no block
    re-quantises exactly, so 16-row fp8_block codes are used and the output
    carries that FP8 rounding; against the reference algorithm (oracle, bf16
    scores of the given values) it stays a close approximation."""
    from low_bit_fake_quant.attention_triton import _requant_qk, fake_quant_attention_triton
    g = torch.Generator().manual_seed(0)
    B, H, S, D = 1, 2, 256, 128
    q = torch.randn(B, H, S, D, generator=g).bfloat16()
    k = torch.randn(B, H, S, D, generator=g).bfloat16()
    v_fp = torch.randn(B, H, S, D, generator=g)
    v_scale = (v_fp.abs().amax(dim=-2) / 448.0).clamp_min(1e-6)
    v_bf16 = (v_fp / v_scale.unsqueeze(-2)).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.bfloat16)
    _, _, blk, exact = _requant_qk(q.to(gpu), 64, S)
    assert not exact and blk == 16
    out = fake_quant_attention_triton(q.to(gpu), k.to(gpu), v_bf16.to(gpu), v_scale.to(gpu), sm_scale=D ** -0.5,
                                      p_max_offset=8, block_m=64, block_n=64).cpu()
    ref = oattn.attention(q, k, v_bf16, v_scale, sm_scale=D ** -0.5, p_max_offset=8, block_m=64, block_n=64)
    c = cosine(out, ref)
    print(f"never-FP8 inputs: cosine vs reference {c:.6f}, max|diff| {(out.float() - ref.float()).abs().max():.3e}")
    assert c > 0.99
