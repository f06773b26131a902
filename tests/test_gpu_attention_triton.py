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
import warnings

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


def _replay_entry(out, q, k, v, v_scale, label, okw, ops, cfg, sm, v_eff=None, stats=None):
    """Strict check of the entry's output against the oracle's restatement of
    the reference kernel (oracle.attention) replayed on the kernel's own scores
    (attention_scores: the FP8-code products plus the qm correction table), with
    the V the kernel actually multiplies (``v_eff`` = (V values, V scale) after
    any re-quantisation).  Returns the replay debug dict."""
    from low_bit_fake_quant.attention_kernel import attention_scores
    u = attention_scores(ops, cfg, sm).reshape(ops.b, ops.h, ops.s, ops.s).cpu()
    vv, vs = v_eff if v_eff is not None else (v.cpu(), v_scale.cpu())
    rep, rstats, dbg = oattn.attention(q.cpu(), k.cpu(), vv, vs, scores_log2=u, return_debug=True,
                                       return_blasst_stats=True, **okw)
    parity.strict_check(out.cpu(), rep, label, allowance=dbg["flip_allowance"])
    if stats is not None and okw.get("blasst_lambda") is not None:
        assert torch.equal(stats.cpu(), rstats)
    return dbg


def _smoothed_study(seed=41, n=1024, h=2, d=128, block=64, qsb=256, vsb=128, v_mode="fp8_channel",
                    v_raw_bf16=False):
    """Inputs the way the reference's smoothing pipeline hands them to the
    kernel: K_s = K - mean_S(K) (bf16), Q_c = Q - qm (256-row group means),
    both fp8_block-quantised and dequantised to bf16; V_c = V - per-block mean
    (v_alpha), FP8-cast per channel (E4M3 values + per-channel scale), as
    fp8_block E4M3 values + block scales, or (v_raw_bf16) left as bf16."""
    from low_bit_fake_quant import fp8_block_dequant, fp8_block_quant
    from low_bit_fake_quant.wan import Workload, make_inputs
    from oracle import preprocess as opre
    from oracle import quant as oq
    q, k, v = make_inputs(Workload("t", h, n, d, None, q_clusters=4, v_bias=True), seed=seed)
    k_s, _ = opre.smooth_k(k)
    q_c, qm = opre.group_mean_q(q, block_q=qsb)
    v_c, v_alpha = opre.smooth_v_per_block(v, block_s=vsb)
    dev = torch.device("cuda:0")
    perm = (0, 2, 1, 3)

    def fq(t):
        c, sc = fp8_block_quant(t.to(dev), block_s=block)
        return fp8_block_dequant(c, sc, block_s=block, dtype=torch.bfloat16).permute(*perm).contiguous()

    x = dict(q=fq(q_c), k=fq(k_s), k_smooth=k_s.permute(*perm).contiguous().to(dev), qm=qm.float().to(dev),
             v_alpha=v_alpha.float().to(dev), sm=1.0 / math.sqrt(d), qsb=qsb, vsb=vsb, block=block)
    if v_raw_bf16:
        x["v"] = v_c.permute(*perm).contiguous().to(dev)
        x["v_scale"] = torch.ones(1, h, d, device=dev)
    elif v_mode == "fp8_channel":
        c, sc = oq.fp8_per_channel_quant(v_c)
        x["v"] = oq.decode(c).to(torch.bfloat16).permute(*perm).contiguous().to(dev)
        x["v_scale"] = sc.float().to(dev)
    else:
        c, sc = oq.fp8_block_quant(v_c, block)
        x["v"] = oq.decode(c).to(torch.bfloat16).permute(*perm).contiguous().to(dev)
        x["v_scale"] = torch.ones(1, h, d, device=dev)
        x["v_block_scale"] = sc.float().contiguous().to(dev)
    return x


ENTRY_CASES = {
    # qm correction (qm_bhgd + k_smooth_bhsd -> the kernel's bias table), online max
    "qm_online_elementwise": dict(p_quant_mode="elementwise", qm=True),
    # + rowmax_est_bhs (group-constant qm_k estimate) with dynamic P (the up/down thresholds)
    "qm_rowmax_est_dynamic": dict(p_quant_mode="dynamic", qm=True, est=True),
    # fixed estimate with mx P
    "qm_rowmax_est_mx": dict(p_quant_mode="mx", qm=True, est=True),
    # V smoothing with per-channel V (v_alpha / v_scale inside the kernel) and dynamic P
    "valpha_channelV_dynamic": dict(p_quant_mode="dynamic", valpha=True),
    # V smoothing with fp8_block V and mx P
    "valpha_blockV_mx": dict(p_quant_mode="mx", valpha=True, v_mode="fp8_block"),
    # V that is not E4M3-valued (pre-dequantised bf16): re-quantised per channel
    "rawV_valpha_elementwise": dict(p_quant_mode="elementwise", valpha=True, raw_v=True),
}


@pytest.mark.parametrize("name", sorted(ENTRY_CASES))
def test_entry_conversions_match_oracle(gpu, name):
    """Each conversion the kernel-level entry does on its own -- the qm
    correction into the kernel's log2 bias table, the rowmax_est_bhs group
    collapse, v_alpha over a per-channel V scale, the mx and dynamic P modes,
    and the per-channel re-quantisation of a V that is not E4M3-valued (its
    scale times v_scale_bhd) -- checked strictly against the oracle's
    restatement of the reference kernel replayed on the kernel's own scores,
    with the V the kernel multiplies."""
    from low_bit_fake_quant.attention_triton import RequantWarning, fake_quant_attention_triton, triton_operands
    from oracle import fp8
    c = ENTRY_CASES[name]
    x = _smoothed_study(v_mode=c.get("v_mode", "fp8_channel"), v_raw_bf16=c.get("raw_v", False))
    kw = dict(sm_scale=x["sm"], p_max_offset=8, block_m=64, block_n=64, p_quant_mode=c["p_quant_mode"])
    if c["p_quant_mode"] == "mx":
        kw["p_mx_block_n"] = 64
    okw = dict(sm_scale=x["sm"], p_max_offset=8, block_m=64, block_n=64, p_quant_mode=c["p_quant_mode"])
    if c.get("qm"):
        kw.update(qm_bhgd=x["qm"], k_smooth_bhsd=x["k_smooth"], q_smooth_block=x["qsb"])
        okw.update(qm=x["qm"].cpu(), k_smooth=x["k_smooth"].cpu(), q_smooth_block=x["qsb"])
    if c.get("est"):
        est = oattn.estimate_rowmax_qm_k(x["qm"].cpu(), x["k_smooth"].cpu().permute(0, 2, 1, 3), block_q=x["qsb"],
                                         sm_scale=x["sm"])
        kw["rowmax_est_bhs"] = est.to(gpu)
        okw["rowmax_est"] = est
    if c.get("valpha"):
        kw.update(v_alpha=x["v_alpha"], v_smooth_block=x["vsb"])
        okw.update(v_alpha=x["v_alpha"].cpu(), v_smooth_block=x["vsb"])
    if "v_block_scale" in x:
        kw.update(v_block_scale_bsh=x["v_block_scale"], v_block_size=x["block"])
        okw.update(v_block_scale=x["v_block_scale"].cpu(), v_block_size=x["block"])
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        out = fake_quant_attention_triton(x["q"], x["k"], x["v"], x["v_scale"], **kw)
        ops, cfg, _ = triton_operands(x["q"], x["k"], x["v"], x["v_scale"], **kw)
    warned = any(issubclass(r.category, RequantWarning) for r in rec)
    assert warned == bool(c.get("raw_v")), "a RequantWarning exactly when an input is re-quantised"
    v_eff = None
    if c.get("raw_v"):
        # the kernel multiplies the per-channel FP8 codes of V with their scale (times v_scale_bhd)
        codes = ops.v_codes_t[..., :ops.s].transpose(-1, -2).cpu().numpy()
        v_eff = (torch.from_numpy(fp8.decode(codes)).to(torch.bfloat16), ops.v_scale.cpu())
    _replay_entry(out, x["q"], x["k"], x["v"], x["v_scale"], name, okw, ops, cfg, x["sm"], v_eff=v_eff)


def test_entry_rejects_zero_v_scale_with_v_alpha(gpu):
    from low_bit_fake_quant.attention_triton import fake_quant_attention_triton
    x = _smoothed_study()
    vs = x["v_scale"].clone()
    vs[0, 0, 5] = 0.0
    with pytest.raises(ValueError, match="finite and > 0"):
        fake_quant_attention_triton(x["q"], x["k"], x["v"], vs, sm_scale=x["sm"], p_max_offset=8,
                                    v_alpha=x["v_alpha"], v_smooth_block=x["vsb"])


def test_values_that_were_never_fp8(gpu):
    """Random bf16 Q/K (as the reference's own kernel test feeds it): no block
    re-quantises exactly, so 16-row fp8_block codes are used (a RequantWarning
    says so) and the output carries that FP8 rounding.  Everything after the
    scores is pinned strictly: the output equals the oracle's restatement of
    the reference kernel replayed on the kernel's own scores (the products of
    those codes) within the north-star tolerance; against the reference
    algorithm on the given bf16 values it stays a close approximation."""
    from low_bit_fake_quant.attention_triton import (RequantWarning, _requant_qk, fake_quant_attention_triton,
                                                     triton_operands)
    g = torch.Generator().manual_seed(0)
    B, H, S, D = 1, 2, 256, 128
    q = torch.randn(B, H, S, D, generator=g).bfloat16()
    k = torch.randn(B, H, S, D, generator=g).bfloat16()
    v_fp = torch.randn(B, H, S, D, generator=g)
    v_scale = (v_fp.abs().amax(dim=-2) / 448.0).clamp_min(1e-6)
    v_bf16 = (v_fp / v_scale.unsqueeze(-2)).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.bfloat16)
    _, _, blk, exact = _requant_qk(q.to(gpu), 64, S)
    assert not exact and blk == 16
    kw = dict(sm_scale=D ** -0.5, p_max_offset=8, block_m=64, block_n=64)
    with pytest.warns(RequantWarning):
        out = fake_quant_attention_triton(q.to(gpu), k.to(gpu), v_bf16.to(gpu), v_scale.to(gpu), **kw).cpu()
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RequantWarning)
        ops, cfg, _ = triton_operands(q.to(gpu), k.to(gpu), v_bf16.to(gpu), v_scale.to(gpu), **kw)
    _replay_entry(out, q, k, v_bf16, v_scale, "never-FP8", dict(kw), ops, cfg, kw["sm_scale"])
    ref = oattn.attention(q, k, v_bf16, v_scale, **kw)
    c = cosine(out, ref)
    print(f"never-FP8 inputs: cosine vs reference {c:.6f}, max|diff| {(out.float() - ref.float()).abs().max():.3e}")
    assert c > 0.99
