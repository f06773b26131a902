"""Parity helpers shared by the GPU attention tests and the smoke check.

The attention kernel is checked in three parts, each against the CPU oracle
(the restatement of the reference path, ``oracle/``):

1. **Scores.**  ``lbfq_attention_scores`` returns the kernel's log2-unit
   scores, formed with the kernel's own MFMA sequence.  They must equal the
   exact scores of the same FP8 codes (float64 products and sums) within the
   accumulation error of the gfx950 FP8 MFMA: measured at <= 3.4e-4 *
   max|a| * max|b| per 32x32x64 MFMA, bounded here by ``MFMA_REL = 2^-10``
   (plus fp32 rounding of the scale products).
2. **Everything after the scores.**  The oracle replays the reference
   algorithm (row max, thresholds, BLASST, P quantisation, PV, V scales,
   smoothing, epilogue; ``attention_triton.py:163-407``) on the kernel's
   scores and row-max estimate.  The kernel's output must match that replay
   within the north-star tolerance: cosine >= 0.9999 and |diff| <= 1e-2 --
   or one bf16 ulp of the value where that is larger (both sides round an
   fp32 result to bf16; at |o| >= 2 one ulp is 1/64).  BLASST skip decisions
   and statistics must match the replay exactly.
3. **Against the reference itself** (the oracle with its own bf16-dequant
   scores, ``attention.py:532-535``), every configuration, BLASST included
   (``reference_bound``): the kernel may not drift from the reference further
   than the reference algorithm moves under either score perturbation that
   separates the two -- its own bf16 rounding of the dequantised Q/K (the
   reference with exact fp32 dequant) or the FP8 MFMA's accumulation error
   (the replay on the kernel's scores against the exact-dequant reference) --
   plus the strict tolerance, element-wise and in angle.  The dense
   configurations must also keep cosine >= 0.9999 against the reference
   wherever the reference itself keeps it against its exact-dequant variant.
   Element-wise agreement to 1e-2 alone is not attainable by an FP8-MFMA
   kernel: the reference rounds the dequantised Q/K to bf16 (up to 2^-9
   relative per operand) and the MFMA accumulates with ~2^-12 relative error;
   both perturb the scores, which flips E4M3 P codes at rounding boundaries
   and moves the P scales and row sums.  Item 2 shows that every difference
   comes from the scores.  BLASST decisions must agree with the reference
   except in rows whose predicate margin is within the score perturbation of
   ln(lambda).
4. **Path A** (``p_requant=False``): ``sdpa_replay`` evaluates the
   reference's SDPA / Q-smoothing attention in float64 on the native path's
   own dequantised operands and bounds the difference element-wise by one
   SDPA-dtype ulp plus the roundings the kernel's fp32 arithmetic may resolve
   the other way.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import fp8
from oracle import pipeline as opipe

COS_MIN = 0.9999
MAXABS = 1e-2
MFMA_REL = 2.0 ** -10
LOG2E = 1.4426950408889634


def cosine(a, b) -> float:
    """Cosine similarity in float64 (a float32 reduction over ~10^6 elements
    is off by ~10^-5, the size of the margins checked here)."""
    a, b = a.double().flatten(), b.double().flatten()
    return ((a @ b) / (a.norm() * b.norm()).clamp_min(1e-300)).item()


def ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    a = x.float().abs().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - 7)


def tolerance(ref: torch.Tensor) -> torch.Tensor:
    """max(1e-2, one bf16 ulp of the reference value), element-wise."""
    return torch.maximum(torch.full(ref.shape, MAXABS), ulp_bf16(ref))


def kernel_operands(q, k, v, cfg, dev, sm_scale=None):
    """The quantised operands exactly as fake_quant_attention builds them."""
    from low_bit_fake_quant.attention import _lazy_preprocess, quantize_operands
    sm = q.shape[-1] ** -0.5 if sm_scale is None else sm_scale
    prep = _lazy_preprocess(q.to(dev), k.to(dev), v.to(dev), cfg)
    return quantize_operands(prep, cfg, sm), sm


def kernel_scores(ops, cfg, sm, rows=None) -> torch.Tensor:
    """(B, H, R, S) log2-unit scores of the kernel (rows in its reordered order), CPU."""
    from low_bit_fake_quant.attention_kernel import attention_scores
    u = attention_scores(ops, cfg, sm, rows=rows)
    return u.reshape(ops.b, ops.h, -1, ops.s).cpu()


def replay(q, k, v, cfg, ops, u, **kw):
    """The oracle's reference algorithm on the kernel's scores and row-max
    estimate; returns (output, ..., debug) with the debug dict last."""
    rm = ops.rowmax.cpu() if ops.rowmax is not None else None
    return opipe.fake_quant_attention(q, k, v, cfg, scores_log2=u, rowmax_log2=rm, return_debug=True, **kw)


def check_against_replay(out, q, k, v, cfg, ops, u, label=""):
    """Replay + strict check; returns (cos, max|diff|, replay output, replay debug)."""
    rep, dbg = replay(q, k, v, cfg, ops, u)
    c, m = strict_check(out, rep, label, allowance=dbg["flip_allowance_nhd"])
    return c, m, rep, dbg


def strict_check(out, rep, label="", allowance=None):
    """North-star tolerance against the replay; returns (cos, max|diff|).
    ``allowance`` (the replay's ``flip_allowance``, same layout as the
    output) adds, per element, the change that one-step flips of P codes
    within 2^-15 of an E4M3 rounding midpoint could cause: codes that the two
    sides' fp32-level differences in evaluating the same scores (hardware
    exp2 and reciprocal vs torch) can round either way.  Elements that need
    it are counted in the message."""
    out, rep = out.float().cpu(), rep.float().cpu()
    fin = torch.isfinite(rep)
    assert torch.equal(torch.isfinite(out), fin), f"{label}: non-finite outputs differ from the replay"
    d = (out - rep).abs()[fin]
    tol = tolerance(rep[fin])
    over = d > tol
    if allowance is not None:
        tol = tol + allowance.float().cpu()[fin]
    bad = d > tol
    c = cosine(out[fin], rep[fin])
    assert c >= COS_MIN and not bad.any(), (
        f"{label}: vs replay cos={c:.7f} max|diff|={d.max():.3e} elements beyond tolerance={int(bad.sum())} "
        f"(beyond 1e-2 / 1 ulp before the flip allowance: {int(over.sum())})")
    if over.any():
        print(f"{label}: {int(over.sum())} elements within the rounding-edge flip allowance")
    return c, d.max().item()


def angle(a, b) -> float:
    """Angle (radians) between two flattened tensors, in float64: unlike
    1 - cosine it obeys the triangle inequality, so gaps can be added."""
    a, b = a.double().flatten(), b.double().flatten()
    c = (a @ b) / (a.norm() * b.norm()).clamp_min(1e-300)
    return math.acos(max(-1.0, min(1.0, c.item())))


def reference_bound(out, ref, ref32, rep, label="", allowance=None):
    """The kernel against the reference itself (the oracle with its own
    bf16-dequant scores, attention.py:532-535), bounded by how far the
    reference algorithm moves under the two score perturbations that separate
    the two, each measured on the same rows:

    * the reference's own: its bf16 rounding of the dequantised Q/K, i.e.
      ``ref32`` (the reference with exact fp32 dequant) against ``ref``;
    * the kernel's: the FP8 MFMA's accumulation error in the scores (bounded
      on its own by test_kernel_scores_match_exact_products), i.e. ``rep``
      (the reference algorithm replayed on the kernel's scores) against
      ``ref32``.

    With G = the larger of the two max-abs gaps:
    * element-wise: |out - ref| <= G + max(1e-2, 1 bf16 ulp of ref) [+ the
      replay's rounding-edge flip allowance];
    * angle(out, ref) <= the larger of the two gaps' angles + acos(0.9999)
      (angles add; 1 - cos does not).
    A kernel whose drift from the reference exceeds the larger single
    perturbation by more than the tolerance fails.  Rows the reference leaves
    non-finite (BLASST rows that skip every block with the zero fill: 0/0)
    are left out.  Returns a dict of the measured quantities."""
    out, ref, ref32, rep = (t.float().cpu() for t in (out, ref, ref32, rep))
    fin = torch.isfinite(out) & torch.isfinite(ref) & torch.isfinite(ref32) & torch.isfinite(rep)
    o, r, r32, rp = out[fin], ref[fin], ref32[fin], rep[fin]
    g_self = (r32 - r).abs().max().item()
    g_mfma = (rp - r32).abs().max().item()
    a_self, a_mfma, a_out = angle(r32, r), angle(rp, r32), angle(o, r)
    d = (o - r).abs()
    tol = tolerance(r) + max(g_self, g_mfma)
    if allowance is not None:
        tol = tol + allowance.float().cpu()[fin]
    bad = d > tol
    res = {"cos_ref": cosine(o, r), "max_abs_ref": d.max().item(), "frac_gt_1e-2_ref": (d > MAXABS).float().mean().item(),
           "cos_ref32": cosine(o, r32), "max_abs_ref32": (o - r32).abs().max().item(),
           "ref_self_cos": cosine(r32, r), "ref_self_max_abs": g_self,
           "mfma_gap_cos": cosine(rp, r32), "mfma_gap_max_abs": g_mfma,
           "elements": int(fin.sum()), "nonfinite_left_out": int((~fin).sum())}
    print(f"{label}: vs reference cos={res['cos_ref']:.7f} max|diff|={res['max_abs_ref']:.3e} | reference's own "
          f"bf16-vs-fp32 gap cos={res['ref_self_cos']:.7f} max={g_self:.3e} | MFMA score-error gap "
          f"cos={res['mfma_gap_cos']:.7f} max={g_mfma:.3e} | vs exact-dequant reference "
          f"cos={res['cos_ref32']:.7f} max={res['max_abs_ref32']:.3e}")
    assert a_out <= max(a_self, a_mfma) + math.acos(COS_MIN), (
        f"{label}: angle to the reference {a_out:.3e} > max(own {a_self:.3e}, MFMA {a_mfma:.3e}) + acos(0.9999)")
    assert not bad.any(), (
        f"{label}: {int(bad.sum())} elements beyond max(|ref32 - ref|, |rep - ref32|) ({max(g_self, g_mfma):.3e}) "
        f"+ tolerance; max|diff| {d.max():.3e}")
    return res


def exact_scores_and_bound(ops, cfg, sm):
    """float64 scores of the kernel's FP8 codes (exact products and sums) and a
    bound on the kernel's error: the MFMA accumulation (MFMA_REL of max|a|max|b|
    and of the accumulator input, per 64-wide MFMA) plus fp32 roundings of the
    scale products and of the qm correction's start value.  (B,H,S,S) each."""
    S, D = ops.s, ops.d
    qc = torch.from_numpy(fp8.decode(ops.q_codes.cpu().numpy())).double()[:, :, :S]
    kc = torch.from_numpy(fp8.decode(ops.k_codes.cpu().numpy())).double()[:, :, :S]
    sml2 = float(np.float32(np.float32(sm) * np.float32(LOG2E)))
    if cfg.qk_quant == "mxfp8":
        qe = torch.from_numpy(ops.q_scale.cpu().numpy().astype(np.int64))[:, :, :S]
        ke = torch.from_numpy(ops.k_scale.cpu().numpy().astype(np.int64))[:, :, :S]
        qv = qc * torch.pow(2.0, (qe - 127).double()).repeat_interleave(32, -1)
        kv = kc * torch.pow(2.0, (ke - 127).double()).repeat_interleave(32, -1)
        C = torch.full((1, 1, S, S), sml2, dtype=torch.float64)
    else:
        blk = cfg.fp8_block_size
        qs = ops.q_scale.cpu().double().repeat_interleave(blk, -1)[:, :, :S]
        ks = ops.k_scale.cpu().double().repeat_interleave(blk, -1)[:, :, :S]
        qv, kv = qc, kc
        C = sml2 * qs[..., :, None] * ks[..., None, :]
    dot = torch.zeros(qv.shape[0], qv.shape[1], S, S, dtype=torch.float64)
    bias = torch.zeros_like(dot)
    if ops.bias is not None:
        g = cfg.q_smooth_block_size
        b = ops.bias.cpu().double()[..., :S]                      # (B,H,G,S)
        bias = b.repeat_interleave(g, 2)[:, :, :S]
    err = torch.zeros_like(dot)
    acc_in = bias / C
    for hh in range(D // 64):
        qh, kh = qv[..., 64 * hh:64 * hh + 64], kv[..., 64 * hh:64 * hh + 64]
        part = torch.matmul(qh, kh.transpose(-2, -1))
        mq, mk = qh.abs().amax(-1), kh.abs().amax(-1)
        err += MFMA_REL * (mq[..., :, None] * mk[..., None, :] + acc_in.abs())
        dot += part
        acc_in = bias / C + dot
    u = dot * C + bias
    bound = err * C + 2.0 ** -20 * (u.abs() + bias.abs()) + 1e-30
    return u, bound


def flipped_codes(dbg_a, dbg_b):
    """Positions whose E4M3 P codes differ between two oracle runs, and whether
    every such pair of codes is one E4M3 step apart with the pre-quantisation
    values on either side of the rounding midpoint between them."""
    ca, cb = dbg_a["codes"], dbg_b["codes"]
    diff = ca != cb
    if not diff.any():
        return diff, True
    va = torch.from_numpy(fp8.decode(ca[diff].numpy())).double()
    vb = torch.from_numpy(fp8.decode(cb[diff].numpy())).double()
    xa, xb = dbg_a["x"][diff].double(), dbg_b["x"][diff].double()
    lo, hi = torch.minimum(va, vb), torch.maximum(va, vb)
    # adjacent magnitudes: no E4M3 value strictly between them
    allv = torch.from_numpy(np.unique(np.abs(fp8.DECODE[~np.isnan(fp8.DECODE)]))).double()
    idx_lo = torch.searchsorted(allv, lo.abs().contiguous())
    idx_hi = torch.searchsorted(allv, hi.abs().contiguous())
    same_sign = (torch.sign(va) == torch.sign(vb)) | (va == 0) | (vb == 0)
    adjacent = ((idx_hi - idx_lo).abs() == 1) & same_sign
    mid = (lo + hi) / 2
    straddle = ((xa - mid) * (xb - mid) <= 0)
    return diff, bool((adjacent & straddle).all())


def skip_agreement(rsk_kernel, dbg_ref, u_kernel, order):
    """Per-row skip counts of the kernel vs the reference (oracle with its own
    scores).  Rows where any block's predicate margin is within twice the
    largest score difference of that row (natural units) are excluded.
    Returns (rows compared, rows excluded, disagreeing compared rows)."""
    s_ref = dbg_ref["s"].double()                       # natural units, reordered rows
    s_ker = u_kernel.double() / LOG2E
    fin = torch.isfinite(s_ref) & torch.isfinite(s_ker)
    gap = torch.where(fin, (s_ref - s_ker).abs(), torch.zeros_like(s_ref)).amax(-1)   # (B,H,R)
    margin = dbg_ref["margin"].double()                 # (B,H,R,blocks)
    near = (margin.abs() < 2 * gap[..., None] + 1e-6).any(-1)
    rs_ref = dbg_ref["row_skips"]
    b, h, r = rs_ref.shape
    rs_ref = rs_ref.reshape(b * h, r)
    near = near.reshape(b * h, r)
    if order is not None:
        rs_o, near_o = torch.empty_like(rs_ref), torch.empty_like(near)
        rs_o.scatter_(1, order.long(), rs_ref)
        near_o.scatter_(1, order.long(), near)
        rs_ref, near = rs_o, near_o
    rsk = rsk_kernel.cpu()
    cmp = ~near
    return int(cmp.sum()), int(near.sum()), int((rsk[cmp] != rs_ref[cmp]).sum())


def sampled_rows(q, k, v, cfg, ops, rows, sm, tail=0, n_real=None, with_ref32=False):
    """Replay and reference for a sample of rows of the kernel's reordered row
    order (full-length checks; every head has its own k-means order).
    ``tail`` adds, for every head, the kernel rows of ``tail`` caller rows
    spread over the last 256 real rows (n_real - 256 .. n_real - 1), so the
    end of the sequence next to the padding is always checked.  Returns
    (caller rows (B*H, R), scores, replay (B,R,H,D), reference (B,R,H,D),
    replay debug[, exact-dequant reference (B,R,H,D)]); the oracle's
    preprocess runs once."""
    qw, kw, vw, qm, v_alpha, q_km, _ = opipe.preprocess(q, k, v, cfg)
    if tail:
        n = n_real if n_real is not None else q.shape[1]
        last = torch.linspace(n - 256, n - 1, tail).round().long()
        if q_km is not None:
            extra = q_km["inverse_order"][:, last].flatten()      # kernel rows of those caller rows, every head
        else:
            extra = last
        rows = torch.cat([rows, extra]).unique()
    rows = rows.sort().values
    if q_km is not None:
        caller = q_km["order"][:, rows]
    else:
        caller = rows.unsqueeze(0).expand(ops.b * ops.h, -1)
    u = kernel_scores(ops, cfg, sm, rows=rows.to(torch.int32))
    rm = ops.rowmax.cpu() if ops.rowmax is not None else None
    rep, dbg_rep = opipe.p_requant_path(qw, kw, vw, qm, v_alpha, cfg, sm, torch.float32, rows=rows,
                                        scores_log2=u, rowmax_log2=rm, return_debug=True)
    ref = opipe.p_requant_path(qw, kw, vw, qm, v_alpha, cfg, sm, torch.float32, rows=rows)
    if not with_ref32:
        return caller, u, rep, ref, dbg_rep
    ref32 = opipe.p_requant_path(qw, kw, vw, qm, v_alpha, cfg, sm, torch.float32, rows=rows,
                                 qk_dequant_dtype=torch.float32)
    return caller, u, rep, ref, dbg_rep, ref32


def gather_caller_rows(out: torch.Tensor, caller: torch.Tensor) -> torch.Tensor:
    """out (B,S,H,D) in caller order -> (B,R,H,D) at each head's caller rows."""
    b, s, h, d = out.shape
    idx = caller.reshape(b, h, -1).permute(0, 2, 1)                       # (B,R,H)
    return torch.gather(out, 1, idx.unsqueeze(-1).expand(-1, -1, -1, d))


def unpermute_rows(t: torch.Tensor, order) -> torch.Tensor:
    """(B*H, S) in reordered row order -> caller row order."""
    if order is None:
        return t
    o = torch.empty_like(t)
    o.scatter_(1, order.long(), t)
    return o


def ulp_dt(x: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """One ulp of the SDPA dtype (bf16: 8 significant bits, fp16: 11) at |x|;
    the spacing of the smallest normal binade below it."""
    bits, tiny = (7, 2.0 ** -126) if dt == torch.bfloat16 else (10, 2.0 ** -14)
    return torch.pow(2.0, torch.floor(torch.log2(x.abs().double().clamp_min(tiny))) - bits)


def _rnd(x: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """x rounded to fp32, then to dt (the kernel rounds fp32 values)."""
    return x.float().to(dt).double()


def sdpa_replay(sops, out: torch.Tensor, sm_scale: float, rows=None) -> dict:
    """Path A's attention (attention.py:288-319) in float64 on the kernel's own
    operands (``SdpaOperands``: Q, K, V^T in the SDPA dtype, the qm.K_s table),
    against the kernel's output ``out`` (NHD, caller row order), optionally
    for a subset of the kernel's query rows (one index vector for every head,
    or a (B*H, R) set per head).

    Element-wise, |out - o64| <= ulp(o64) + A.  The ulp covers the output's
    rounding to the SDPA dtype; A is what the kernel's fp32 arithmetic may
    legitimately move:

    * no qm (SDPA, P in fp32): every score carries the fp32 accumulation error
      D 2^-24 sum|q||k| (times sm_scale) and every P a relative error below
      2^-15 (its two-term SDPA-dtype representation, exp2): A = 2 max|v|
      sum_j p_j (e^delta_j - 1) + S 2^-24 p.|v| + eps_l |o|, with eps_l =
      (S/64 + 64) 2^-24 the relative error of the row sum (about S/64
      rescaled tile sums of 32 terms per lane);
    * qm branch: the main score is rounded to the SDPA dtype (attention.py:314)
      and P is rounded after the normalisation (:318).  Where the float64 main
      score lies within the fp32 accumulation error of a rounding boundary,
      the kernel may round it one ulp the other way: those scores add
      2 max|v| p_j (e^(ulp sm) - 1) to A, and they shift every other P of the
      row by the same relative amount, which widens the window (2^-16
      relative, plus eps_l, plus that shift) inside which a P may round the other way,
      adding ulp(p_i)|v_i| for each such P.

    Returns the largest |diff| / bound ("excess", <= 1 passes), the fraction
    of elements equal to the rounded float64 value, the largest |diff| and the
    counts of boundary cases."""
    dt = sops.q.dtype
    b, h, s, d = sops.b, sops.h, sops.s, sops.d
    ridx = torch.arange(s) if rows is None else torch.as_tensor(rows).long()
    # kernel rows per (b, h): one set for every head, or (B*H, R) sets
    ridx = (ridx.expand(b * h, -1) if ridx.ndim == 1 else ridx).reshape(b, h, -1)

    def take(t):  # (B,H,S,X) -> (B,H,R,X) at the kernel rows
        return torch.gather(t, 2, ridx.unsqueeze(-1).expand(-1, -1, -1, t.shape[-1]))

    q = take(sops.q[:, :, :s].cpu().double())
    k = sops.k[:, :, :s].cpu().double()
    v = sops.v_t[..., :s].cpu().double().transpose(-1, -2)                 # (B,H,S,D)
    o = out.cpu().double().permute(0, 2, 1, 3)                              # output-row order
    if sops.out_row_map is not None:
        order = sops.out_row_map.cpu().long().reshape(b, h, s)
        o = torch.gather(o, 2, order.unsqueeze(-1).expand(-1, -1, -1, d))  # kernel row order
    o = take(o)
    main = q @ k.transpose(-1, -2)
    err_main = d * 2.0 ** -24 * (q.abs() @ k.abs().transpose(-1, -2))
    vabs = v.abs()
    vmax = vabs.amax(dim=2, keepdim=True)                                   # (B,H,1,D)
    acc_err = s * 2.0 ** -24
    # the row sum accumulates ~S/64 rescaled tile sums of 32 terms per lane
    l_err = (s / 64 + 64) * 2.0 ** -24
    info = {}
    if sops.bias is None:
        p = torch.softmax(main * sm_scale, dim=-1)
        o64 = p @ v
        delta = sm_scale * err_main + 2.0 ** -15
        allow = 2 * vmax * (p * torch.expm1(delta)).sum(-1, keepdim=True) + acc_err * (p @ vabs) + l_err * o64.abs()
    else:
        g = sops.bias.shape[2]
        grp = (ridx // sops.q_group).clamp_max(g - 1)                      # (B,H,R)
        bias = torch.gather(sops.bias.cpu()[..., :s], 2, grp.unsqueeze(-1).expand(-1, -1, -1, s)).double()
        main_r = _rnd(main, dt)
        amb_m = _rnd(main - err_main, dt) != _rnd(main + err_main, dt)
        u = main_r * (sm_scale * LOG2E) + bias                              # log2 units
        p = torch.softmax(u * math.log(2.0), dim=-1)
        p_r = _rnd(p, dt)
        shift = (amb_m * p * torch.expm1(ulp_dt(main, dt) * sm_scale)).sum(-1, keepdim=True)
        rel = 2.0 ** -16 + l_err + shift
        amb_p = _rnd(p * (1 - rel), dt) != _rnd(p * (1 + rel), dt)
        o64 = p_r @ v
        allow = 2 * vmax * shift + (amb_p * ulp_dt(p, dt)) @ vabs + acc_err * (p_r @ vabs)
        info = dict(frac_main_boundary=amb_m.double().mean().item(), frac_p_boundary=amb_p.double().mean().item())
    bound = ulp_dt(o64, dt) + allow
    diff = (o - o64).abs()
    return dict(excess=(diff / bound).max().item(), frac_equal=(o == _rnd(o64, dt)).double().mean().item(),
                max_abs=diff.max().item(), **info)


__all__ = ["COS_MIN", "MAXABS", "MFMA_REL", "cosine", "ulp_bf16", "tolerance", "kernel_operands", "kernel_scores",
           "replay", "strict_check", "check_against_replay", "angle", "reference_bound",
           "exact_scores_and_bound", "flipped_codes",
           "skip_agreement", "sampled_rows", "gather_caller_rows", "unpermute_rows",
           "ulp_dt", "sdpa_replay", "math"]
