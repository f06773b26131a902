"""Pins the attention oracle (reference attention_triton.py:109-407,
attention.py:366-395) with checks that do not restate its formulas.

Exact-P construction: with ``sm_scale = ln 2`` and integer dot products, every
score in log2 units is an integer (to fp32 rounding), so every P value is a
power of two.  Powers of two within the covered range are exact E4M3 codes in
all three P modes (elementwise P*2^8, mx pow2 scale, dynamic rowamax/448), so
the streaming K-loop must then reproduce the dense float64 softmax exactly up
to fp32 arithmetic and the final bf16 rounding.  A dropped alpha rescale, a
wrong l update, a transposed operand or a wrong V scale breaks that.  The
BLASST fills are pinned by closed forms: on key blocks of constant score the
max / mean / logn / sample8 / uta fills with alpha 1 reproduce the exact p
(bitwise equal to BLASST off); a block layout whose skip set is known by
construction pins zero / thr fills and the skip statistics.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oattn
from oracle import fp8

LN2 = math.log(2.0)


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp at |x| (spacing of the bf16 grid)."""
    ax = x.abs().clamp_min(2.0 ** -126)
    e = torch.floor(torch.log2(ax))
    return torch.pow(2.0, e - 7)


def _exact_case(s=256, d=64, seed=0, lo=-7, hi=7, h=2):
    """q, k with integer dot products in [lo, hi]; v = E4M3 values; channel scale."""
    g = torch.Generator().manual_seed(seed)
    q = torch.zeros(1, h, s, d)
    k = torch.zeros(1, h, s, d)
    # score = a_i * c_j + b_i * d_j with a,b in {0, 1}, c,d small integers
    a = torch.randint(0, 2, (h, s), generator=g).float()
    b = 1.0 - a
    q[0, :, :, 0], q[0, :, :, 1] = a, b
    c = torch.randint(lo, hi + 1, (h, s), generator=g).float()
    dd = torch.randint(lo, hi + 1, (h, s), generator=g).float()
    k[0, :, :, 0], k[0, :, :, 1] = c, dd
    codes = torch.randint(0, 256, (1, h, s, d), generator=g, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes
    v = torch.from_numpy(fp8.decode(codes.numpy())).float()
    v_scale = torch.rand(1, h, d, generator=g) + 0.5
    return q.bfloat16(), k.bfloat16(), v.bfloat16(), v_scale


def _dense(q, k, v_eff, *, extra=None):
    """float64 softmax with log2-unit integer scores: O = sum 2^s v / sum 2^s."""
    s2 = torch.matmul(q.double(), k.double().transpose(-2, -1))
    if extra is not None:
        s2 = s2 + extra
    w = torch.pow(2.0, s2 - s2.amax(-1, keepdim=True))
    return torch.matmul(w, v_eff.double()) / w.sum(-1, keepdim=True)


def _assert_close_bf16(out, ref, ulps=1.0):
    out = out.double()
    tol = ulps * _bf16_ulp(ref.float()).double() + 1e-6
    err = (out - ref).abs()
    assert (err <= tol).all(), f"max err {err.max().item():.3e} (tol at argmax {tol.flatten()[err.argmax()].item():.3e})"


@pytest.mark.parametrize("p_mode", ["elementwise", "mx", "dynamic"])
@pytest.mark.parametrize("s", [256, 200])  # 200: ragged last key block (masked columns)
def test_exact_p_online_rowmax_equals_dense_softmax(p_mode, s):
    q, k, v, vs = _exact_case(s=s, seed=1)
    out = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode=p_mode)
    ref = _dense(q, k, v.double() * vs.double()[:, :, None, :])
    _assert_close_bf16(out, ref)


def test_exact_p_rises_across_blocks_exercises_alpha():
    """Scores increase block by block, so every block raises the running max."""
    q, k, v, vs = _exact_case(s=256, seed=2, lo=0, hi=0)
    ramp = torch.arange(256) // 64 * 2 - 3.0    # -3, -1, 1, 3 per 64-key block
    k = k.float()
    k[0, :, :, 0] = ramp
    k[0, :, :, 1] = ramp
    k = k.bfloat16()
    for p_mode in ("elementwise", "mx", "dynamic"):
        out = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode=p_mode)
        ref = _dense(q, k, v.double() * vs.double()[:, :, None, :])
        _assert_close_bf16(out, ref)


def test_exact_p_qm_correction_and_fixed_estimate():
    """qm correction (qm . K_s * sm_scale) and the qm_k fixed row max (elementwise P)."""
    q, k, v, vs = _exact_case(s=256, seed=3, lo=-3, hi=3)
    g = torch.Generator().manual_seed(4)
    d = q.shape[-1]
    ks = torch.zeros(1, 2, 256, d)
    ks[0, :, :, 2] = torch.randint(-2, 3, (2, 256), generator=g).float()
    qm = torch.zeros(1, 2, 2, d)            # (B, G, H, D), q_smooth_block 128
    qm[0, :, :, 2] = torch.tensor([[1.0, -1.0], [2.0, 0.0]])
    corr = torch.einsum("bghd,bhnd->bhgn", qm.double(), ks.double()).repeat_interleave(128, dim=2)
    ref = _dense(q, k, v.double() * vs.double()[:, :, None, :], extra=corr)
    for p_mode in ("elementwise", "mx", "dynamic"):
        out = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode=p_mode,
                              k_smooth=ks.bfloat16(), qm=qm, q_smooth_block=128)
        _assert_close_bf16(out, ref)
    # qm_k estimate: brute-force max over keys of the correction, per group
    est = oattn.estimate_rowmax_qm_k(qm, ks.permute(0, 2, 1, 3), block_q=128, sm_scale=LN2)
    brute = torch.zeros(1, 2, 256)
    for hh in range(2):
        for gg in range(2):
            m = max(float(qm[0, gg, hh].double() @ ks[0, hh, n].double()) for n in range(256))
            brute[0, hh, gg * 128:(gg + 1) * 128] = m * LN2
    assert torch.allclose(est, brute, rtol=0, atol=1e-6)
    # fixed estimate at or above the true row max: elementwise P stays exact
    s_full = torch.matmul(q.double(), k.double().transpose(-2, -1)) + corr
    rmax = (s_full.amax(-1) * LN2).float()
    for bump in (0.0, 2.0 * LN2):
        out = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode="elementwise",
                              k_smooth=ks.bfloat16(), qm=qm, q_smooth_block=128, rowmax_est=rmax + bump)
        _assert_close_bf16(out, ref)


@pytest.mark.parametrize("est_shift", [0.0, -20.0, 40.0])
def test_exact_p_qmk_dynamic_thresholds(est_shift):
    """Dynamic P with the qm_k estimate: under-estimates by > 16 (log2) move the
    max up, over-estimates by > 32 move it down; P_deq = p exactly either way."""
    q, k, v, vs = _exact_case(s=256, seed=5)
    ref = _dense(q, k, v.double() * vs.double()[:, :, None, :])
    s_full = torch.matmul(q.double(), k.double().transpose(-2, -1))
    est = ((s_full.amax(-1) + est_shift) * LN2).float()
    qm = torch.zeros(1, 2, 2, q.shape[-1])
    out = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode="dynamic",
                          k_smooth=torch.zeros_like(k), qm=qm, q_smooth_block=128, rowmax_est=est)
    _assert_close_bf16(out, ref)


def test_exact_p_v_block_scale_and_v_smoothing():
    q, k, v, vs = _exact_case(s=256, seed=6)
    g = torch.Generator().manual_seed(7)
    vbs = torch.rand(1, 2, 2, generator=g) + 0.5               # (B, H, S/128)... per reference (B, S/vb, H)
    vbs_bsh = vbs.permute(0, 2, 1).contiguous()                 # (B, S/128, H)
    alpha_v = torch.randn(1, 4, 2, v.shape[-1], generator=g)     # (B, S/64, H, D)
    v_eff = v.double() * vbs.double().repeat_interleave(128, dim=2)[..., None]
    v_eff = v_eff + alpha_v.double().permute(0, 2, 1, 3).repeat_interleave(64, dim=2)
    ref = _dense(q, k, v_eff)
    for p_mode in ("elementwise", "mx", "dynamic"):
        out = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode=p_mode,
                              v_block_scale=vbs_bsh, v_block_size=128, v_alpha=alpha_v, v_smooth_block=64)
        _assert_close_bf16(out, ref, ulps=2.0)


@pytest.mark.parametrize("p_mode", ["elementwise", "mx", "dynamic"])
def test_v_smoothing_accumulator_equals_unsmoothed_v(p_mode):
    """Linearity with non-exact P: P_deq (V + alpha) == P_deq V + rowsum(P_deq) alpha,
    so V smoothing with its C accumulator equals attention on V + alpha
    (the V-smoothing identity of the reference, attention_triton.py:376-383)."""
    g = torch.Generator().manual_seed(12)
    q = torch.randn(1, 2, 256, 64, generator=g).bfloat16()
    k = (torch.randn(1, 2, 256, 64, generator=g) * 2).bfloat16()
    v = torch.randn(1, 2, 256, 64, generator=g).bfloat16()
    alpha_v = torch.randn(1, 4, 2, 64, generator=g) * 3      # (B, S/64, H, D)
    vs = torch.ones(1, 2, 64)
    a = oattn.attention(q, k, v, vs, sm_scale=0.2, p_max_offset=8, p_quant_mode=p_mode, v_alpha=alpha_v,
                        v_smooth_block=64)
    v_full = v.float() + alpha_v.permute(0, 2, 1, 3).repeat_interleave(64, dim=2)
    b = oattn.attention(q, k, v_full, vs, sm_scale=0.2, p_max_offset=8, p_quant_mode=p_mode)
    _assert_close_bf16(a, b.double(), ulps=2.0)


def test_mx_p_ignores_p_max_offset_bitwise():
    """Reference test_v_quant_variants.py:337-356: mx P output is independent of p_max_offset."""
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 2, 192, 64, generator=g).bfloat16()
    k = torch.randn(1, 2, 192, 64, generator=g).bfloat16()
    v = torch.randn(1, 2, 192, 64, generator=g).bfloat16()
    vs = torch.ones(1, 2, 64)
    o0 = oattn.attention(q, k, v, vs, sm_scale=0.125, p_max_offset=0, p_quant_mode="mx")
    o8 = oattn.attention(q, k, v, vs, sm_scale=0.125, p_max_offset=8, p_quant_mode="mx")
    assert torch.equal(o0, o8)


def _constant_block_case(seed=9, s=256, d=64):
    """Keys constant within each 64-key block (per head); random integer levels."""
    g = torch.Generator().manual_seed(seed)
    q = torch.zeros(1, 2, s, d)
    q[0, :, :, 0] = torch.randint(1, 3, (2, s), generator=g).float()
    lev = torch.randint(-4, 5, (2, s // 64), generator=g).float()
    k = torch.zeros(1, 2, s, d)
    k[0, :, :, 0] = lev.repeat_interleave(64, dim=1)
    codes = torch.randint(0, 126, (1, 2, s, d), generator=g, dtype=torch.uint8)
    v = torch.from_numpy(fp8.decode(codes.numpy())).float().bfloat16()
    return q.bfloat16(), k.bfloat16(), v, torch.ones(1, 2, d)


@pytest.mark.parametrize("fill", ["max", "mean", "logn", "sample8", "uta16", "uta", "uta64"])
@pytest.mark.parametrize("p_mode", ["elementwise", "dynamic"])
def test_blasst_exact_fills_on_constant_blocks(fill, p_mode):
    q, k, v, vs = _constant_block_case()
    base = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode=p_mode)
    out, st = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode=p_mode,
                              blasst_lambda=0.3, blasst_fill_mode=fill, blasst_fill_alpha=1.0,
                              blasst_uta_bins=8, return_blasst_stats=True)
    assert st[..., 0].sum() > 0, "the case must make BLASST skip"
    assert torch.equal(out, base)


def test_blasst_never_skips_at_tiny_lambda():
    g = torch.Generator().manual_seed(10)
    q, k, v = (torch.randn(1, 2, 256, 64, generator=g).bfloat16() for _ in range(3))
    vs = torch.ones(1, 2, 64)
    base = oattn.attention(q, k, v, vs, sm_scale=0.125, p_max_offset=8, p_quant_mode="dynamic")
    out, st = oattn.attention(q, k, v, vs, sm_scale=0.125, p_max_offset=8, p_quant_mode="dynamic",
                              blasst_lambda=1e-30, blasst_fill_mode="mean_a1.5", return_blasst_stats=True)
    assert st[..., 0].sum() == 0 and st[..., 1].sum() == 2 * 256 * 4
    assert torch.equal(out, base)


def _dominant_first_block(s=256, d=64, seed=11):
    """Block 0 scores +7 (log2), every later block -7: with lambda = 1e-3
    (ln = -6.9 nats; the gap is 14 log2 = 9.7 nats) every later block is
    skipped for every row."""
    g = torch.Generator().manual_seed(seed)
    q = torch.zeros(1, 1, s, d)
    q[0, 0, :, 0] = 1.0
    k = torch.zeros(1, 1, s, d)
    k[0, 0, :, 0] = -7.0
    k[0, 0, :64, 0] = 7.0
    codes = torch.randint(0, 126, (1, 1, s, d), generator=g, dtype=torch.uint8)
    v = torch.from_numpy(fp8.decode(codes.numpy())).float()
    return q.bfloat16(), k.bfloat16(), v.bfloat16(), torch.ones(1, 1, d)


def test_blasst_zero_and_thr_fill_closed_forms():
    q, k, v, vs = _dominant_first_block()
    lam = 1e-3
    out, st = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode="elementwise",
                              blasst_lambda=lam, blasst_fill_mode="zero", return_blasst_stats=True, block_m=64)
    # every row skips the 3 later blocks: stats per 64-row block = [64*3, 64*4]
    assert torch.equal(st[:, 0, 0], torch.full((4,), 192.0)) and torch.equal(st[:, 0, 1], torch.full((4,), 256.0))
    ref0 = v[0, 0, :64].double().mean(0)
    _assert_close_bf16(out[0, 0], ref0.expand(256, -1))
    # thr: each skipped key gets p = alpha * lambda * 2^offset (pre-quant, in l),
    # quantised elementwise to E4M3 for PV
    a = 0.5
    out_t = oattn.attention(q, k, v, vs, sm_scale=LN2, p_max_offset=8, p_quant_mode="elementwise",
                            blasst_lambda=lam, blasst_fill_mode=f"thr_a{a}")
    pf = float(np.float32(a * lam) * np.float32(256.0))
    pq = float(fp8.decode(fp8.encode(np.array([pf], dtype=np.float32)))[0])
    num = 256.0 * v[0, 0, :64].double().sum(0) + pq * v[0, 0, 64:].double().sum(0)
    den = 256.0 * 64 + pf * 192
    _assert_close_bf16(out_t[0, 0], (num / den).expand(256, -1))


def test_parse_blasst_fill_spellings():
    P = oattn.parse_blasst_fill
    assert P(None, alpha=1.0, uta_bins=16) == (oattn.FILL_ZERO, 1.0, 1)
    assert P("max_a0.25", alpha=1.0, uta_bins=16) == (oattn.FILL_MAX, 0.25, 1)
    assert P("sample8_a2", alpha=1.0, uta_bins=16) == (oattn.FILL_SAMPLE8, 2.0, 1)
    assert P("uta", alpha=3.0, uta_bins=8) == (oattn.FILL_UTA, 3.0, 8)
    assert P("uta16_a1.5", alpha=1.0, uta_bins=8) == (oattn.FILL_UTA, 1.5, 16)
    with pytest.raises(ValueError, match="unknown blasst_fill_mode"):
        P("median", alpha=1.0, uta_bins=16)


# ---- replay on supplied scores, forced P codes, rounding-edge allowance ------------


@pytest.mark.parametrize("p_mode", ["elementwise", "mx", "dynamic"])
def test_supplied_log2_scores_replace_the_score_computation(p_mode):
    """scores_log2 stands in for q.k * sm_scale (+ correction): integer log2
    scores plus an arbitrary integer per-(row, key) term reproduce the dense
    float64 softmax, whatever q and k hold."""
    q, k, v, vs = _exact_case(s=200, seed=21, lo=-5, hi=5)
    g = torch.Generator().manual_seed(5)
    # scores stay within [-6, 6], so every P (>= 2^(8-12)) is a normal E4M3 value
    extra = torch.randint(-1, 2, (1, 2, 200, 200), generator=g).double()
    u = torch.matmul(q.double(), k.double().transpose(-2, -1)) + extra
    junk_q, junk_k = torch.randn(q.shape, generator=g).bfloat16(), torch.randn(k.shape, generator=g).bfloat16()
    out = oattn.attention(junk_q, junk_k, v, vs, sm_scale=0.37, p_max_offset=8, p_quant_mode=p_mode,
                          scores_log2=u.float())
    ref = _dense(q, k, v.double() * vs.double()[:, :, None, :], extra=extra)
    _assert_close_bf16(out, ref)


def test_forced_codes_change_the_output_by_their_value_change():
    """force_codes replaces P codes before dequantisation: with exact
    (power-of-two) P, moving the codes of one key in every row by one E4M3
    step changes each output row by (new - old) * v_key / l exactly (l, the
    pre-quantisation row sum, is unchanged)."""
    q, k, v, vs = _exact_case(s=128, seed=22)
    kw = dict(sm_scale=LN2, p_max_offset=8, p_quant_mode="elementwise")
    out, dbg = oattn.attention(q, k, v, vs, return_debug=True, **kw)
    codes = dbg["codes"].clone()
    mask = torch.zeros_like(codes, dtype=torch.bool)
    j = 37
    mask[..., j] = True
    new = codes.clone()
    new[..., j] = torch.where(codes[..., j] == 0, codes[..., j], codes[..., j] + 1)  # one step up (finite codes)
    out2 = oattn.attention(q, k, v, vs, force_codes=(new, mask), **kw)
    old_v = torch.from_numpy(fp8.decode(codes[..., j].numpy())).double()
    new_v = torch.from_numpy(fp8.decode(new[..., j].numpy())).double()
    l = dbg["x"].double().sum(-1)          # elementwise: p in code units is p itself
    vj = (v.double() * vs.double()[:, :, None, :])[:, :, j, :]                     # (B,H,D)
    expect = out.double() + ((new_v - old_v) / l)[..., None] * vj[:, :, None, :]
    _assert_close_bf16(out2, expect, ulps=1.0)


def test_rounding_edge_step():
    """The E4M3 step at a rounding midpoint within 2^-15 of |x|, else 0."""
    mid = 1.0625                                              # between 1.0 and 1.125
    x = torch.tensor([mid * (1 + 2.0 ** -17), mid * (1 - 2.0 ** -17), mid * (1 + 2.0 ** -12), 1.0, 448.0,
                      2.0 ** -10, -mid * (1 + 2.0 ** -18), 240.0, 232.0 * (1 + 2.0 ** -20)], dtype=torch.float32)
    got = oattn.rounding_edge_step(x)
    want = torch.tensor([0.125, 0.125, 0.0, 0.0, 0.0, 2.0 ** -9, 0.125, 0.0, 16.0])
    assert torch.equal(got, want)


def test_flip_allowance_bounds_flips_of_edge_codes():
    """Scores placed so that many P values sit on E4M3 rounding midpoints
    (u = log2(1.0625) + integer): flipping every such code to its other
    neighbour moves each output by no more than the reported allowance, and
    the allowance is zero where no code is at an edge."""
    q, k, v, vs = _exact_case(s=128, seed=23)
    u = torch.matmul(q.double(), k.double().transpose(-2, -1))
    g = torch.Generator().manual_seed(7)
    edge = torch.rand(u.shape, generator=g) < 0.3
    u = (u + torch.where(edge, torch.tensor(math.log2(1.0625)), torch.tensor(0.0))).float()
    kw = dict(sm_scale=LN2, p_max_offset=8, p_quant_mode="elementwise", scores_log2=u)
    out, dbg = oattn.attention(q, k, v, vs, return_debug=True, **kw)
    step = oattn.rounding_edge_step(dbg["x"])
    assert (step > 0).float().mean() > 0.02   # (rows whose max sits on an edge shift off it)
    vals = torch.from_numpy(fp8.decode(dbg["codes"].numpy())).double()
    x = dbg["x"].double()
    # the other neighbour of each edge value
    other = torch.where(vals >= x, vals - step.double(), vals + step.double()).float()
    flip = torch.from_numpy(fp8.encode(other.numpy()))
    out2 = oattn.attention(q, k, v, vs, force_codes=(flip, step > 0), **kw)
    alw = dbg["flip_allowance"]
    err = (out2.double() - out.double()).abs()
    assert (err <= alw.double() + 2 * _bf16_ulp(out.float()).double()).all()
    out0, dbg0 = oattn.attention(q, k, v, vs, return_debug=True, sm_scale=LN2, p_max_offset=8,
                                 p_quant_mode="elementwise")
    assert dbg0["flip_allowance"].abs().max() == 0.0


@pytest.mark.parametrize("block_n", [64, 128])
def test_rowmax_init_at_the_row_max_equals_the_fixed_estimate(block_n):
    """rowmax_init (attention_triton.py:127-130) starts the online max; at the
    true row max the max never moves (alpha = 1), so the output equals the
    fixed-estimate path (attention_triton.py:212-214) with the same values,
    bit for bit; a start below every score equals the plain online max."""
    q, k, v, v_scale = _exact_case(s=256, d=64, seed=7)
    sm = 1.0
    rm = (torch.matmul(q.float(), k.float().transpose(-2, -1)) * sm).amax(-1)   # (B,H,S)
    kw = dict(sm_scale=sm, p_max_offset=8, block_m=block_n, block_n=block_n, p_quant_mode="elementwise")
    o_init = oattn.attention(q, k, v, v_scale, rowmax_init=rm, **kw)
    o_est = oattn.attention(q, k, v, v_scale, rowmax_est=rm, **kw)
    assert torch.equal(o_init, o_est)
    o_low = oattn.attention(q, k, v, v_scale, rowmax_init=torch.full_like(rm, -1e4), **kw)
    o_online = oattn.attention(q, k, v, v_scale, **kw)
    assert torch.equal(o_low, o_online)

