"""CPU restatement of the P-requant attention kernel (test infrastructure only).

``attention`` follows the K-loop of ``_fake_quant_attn_fwd_kernel``
(``attention_triton.py:109-407``) and the guards / fill parsing of
``fake_quant_attention_triton`` (``attention_triton.py:463-714``); rows are
processed all at once (rows are independent in that kernel) and the loop
runs over K-blocks of ``block_n`` exactly as the reference does:

* scores ``s = (q_deq . k_deq) * sm_scale`` in fp32, plus the qm correction
  ``(qm[group] . K_smooth) * sm_scale`` (lines 154-160); masked columns -inf;
* row max: online (215-217), ``qm_k`` estimate with the dynamic-P
  up/down thresholds 16/32 (log2 units) or the fixed estimate (176-214),
  BLASST predicate (165-175);
* ``p = exp2((s - m) * log2e [+ p_max_offset for elementwise])`` (219-230);
* BLASST fills zero/max/mean/logn/sample8/thr/uta (231-324);
* ``l = l * alpha + sum(p)`` on the pre-quant p (326);
* P quant elementwise / mx / dynamic (329-360);
* ``pv = p_deq @ v``, fp8_block V scale per block (363-372), ``acc`` and the
  V-smoothing accumulator (376-383);
* epilogue ``(acc * v_scale[d] | acc) (+ c) / l`` (387-402) and BLASST stats
  per ``block_m`` rows (404-407).

Tensors are BHSD torch CPU tensors; q/k are the bf16 dequantised values, v is
FP8 values held in bf16 (fp8_channel / fp8_block) or the pre-dequantised
bf16 V (mxfp8), exactly as the reference marshals them
(``attention.py:554-575``).  ``rows`` restricts the computation to a subset
of query rows (used for the bounded CPU baseline sample).

Pinned by ``tests/test_oracle_attention.py`` with checks that do not restate
these formulas: on inputs whose log2-unit scores are integers every P value is
a power of two and exactly representable in all three P modes, so the
streaming loop must reproduce a dense float64 softmax (online row max, rising
row max, qm correction, fixed and dynamic qm_k estimates with both threshold
moves, fp8_block V scales, V smoothing, ragged S); V smoothing equals attention
on V + alpha (linearity, non-exact P); mx P is bitwise independent of
``p_max_offset`` (reference test_v_quant_variants.py:337-356); BLASST fills
reproduce the exact p on constant-score key blocks, zero / thr fills and skip
statistics match closed forms on a block layout whose skip set is known; the
qm_k estimate equals a brute-force maximum.
"""

from __future__ import annotations

import math
import re

import numpy as np
import torch

from . import fp8
from .quant import ceil_log2_exact

LOG2E = 1.4426950408889634
FP8_MAX = 448.0

FILL_ZERO, FILL_MAX, FILL_MEAN, FILL_LOGN, FILL_SAMPLE8, FILL_THR, FILL_UTA = range(7)


def parse_blasst_fill(mode, *, alpha: float, uta_bins: int):
    """``attention_triton.py:674-714``."""
    if mode is None or mode == "zero":
        return FILL_ZERO, float(alpha), 1
    if mode == "max":
        return FILL_MAX, float(alpha), 1
    if mode.startswith("max_a"):
        return FILL_MAX, float(mode[len("max_a"):]), 1
    if mode == "mean":
        return FILL_MEAN, float(alpha), 1
    if mode.startswith("mean_a"):
        return FILL_MEAN, float(mode[len("mean_a"):]), 1
    if mode == "logn":
        return FILL_LOGN, float(alpha), 1
    if mode == "sample8":
        return FILL_SAMPLE8, float(alpha), 1
    if mode.startswith("sample8_a"):
        return FILL_SAMPLE8, float(mode[len("sample8_a"):]), 1
    if mode == "thr":
        return FILL_THR, float(alpha), 1
    if mode.startswith("thr_a"):
        return FILL_THR, float(mode[len("thr_a"):]), 1
    if mode == "uta":
        if uta_bins <= 0:
            raise ValueError(f"blasst_uta_bins must be > 0; got {uta_bins}")
        return FILL_UTA, float(alpha), int(uta_bins)
    m = re.fullmatch(r"uta(\d+)(?:_a([0-9]+(?:\.[0-9]+)?))?", mode)
    if m:
        bins = int(m.group(1))
        if bins <= 0:
            raise ValueError(f"UTA bin count must be > 0; got {bins}")
        a = float(m.group(2)) if m.group(2) is not None else float(alpha)
        return FILL_UTA, a, bins
    raise ValueError(f"unknown blasst_fill_mode: {mode!r}")


def _e4m3_sat(x: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(fp8.round_to_e4m3(x.contiguous().numpy()))


def _f32(x: float) -> torch.Tensor:
    return torch.tensor(x, dtype=torch.float32)


_E4M3_MAG = np.unique(np.abs(fp8.DECODE[~np.isnan(fp8.DECODE)])).astype(np.float64)   # 0 .. 448, sorted
EDGE_REL = 2.0 ** -15


def rounding_edge_step(x: torch.Tensor, rel: float = EDGE_REL) -> torch.Tensor:
    """Per element of x (P in code units): the E4M3 step between the two codes
    around x when |x| lies within rel * |x| of the rounding midpoint between
    them (a value whose code a relative change of rel can flip), else 0."""
    a = np.abs(x.double().numpy())
    i = np.clip(np.searchsorted(_E4M3_MAG, a), 1, len(_E4M3_MAG) - 1)
    lo, hi = _E4M3_MAG[i - 1], _E4M3_MAG[i]
    near = (np.abs(a - (lo + hi) / 2) <= rel * a) & (a < 448.0)
    return torch.from_numpy(np.where(near, hi - lo, 0.0)).float()


def estimate_rowmax_qm_k(qm: torch.Tensor, k_work: torch.Tensor, *, block_q: int, sm_scale: float) -> torch.Tensor:
    """``attention.py:366-395``: (B,H,S) fp32 = max_n(qm[g] . K_s[n]) * sm_scale."""
    qm_b = qm.permute(0, 2, 1, 3).float()                 # (B,H,G,D)
    k_b = k_work.permute(0, 2, 1, 3).float()              # (B,H,S,D)
    g = torch.matmul(qm_b, k_b.transpose(-2, -1)).amax(dim=-1)
    return (g * _f32(sm_scale)).repeat_interleave(block_q, dim=2).contiguous()


def attention(q, k, v, v_scale, *, sm_scale, p_max_offset, block_m=64, block_n=64,
              v_alpha=None, v_smooth_block=0, k_smooth=None, qm=None, q_smooth_block=0,
              v_block_scale=None, v_block_size=0, p_quant_mode="elementwise",
              rowmax_est=None, rowmax_init=None, blasst_lambda=None, blasst_fill_mode="zero",
              blasst_fill_alpha=1.0, blasst_uta_bins=16, return_blasst_stats=False,
              rows=None, return_debug=False, scores_log2=None, force_codes=None):
    """``scores_log2`` (B,H,R,S), when given, replaces the score computation
    (q.k * sm_scale + the qm correction, lines 150-162) by supplied scores in
    log2 units (s = u / log2 e); everything after the scores runs unchanged.
    ``force_codes`` = (codes (B,H,R,S) uint8, mask (B,H,R,S) bool) replaces the
    E4M3 P codes at the masked positions before dequantisation.
    ``return_debug`` adds a dict with the per-block skip masks, the scores
    ``s`` (B,H,R,S, natural units), the P codes (B,H,R,S), their
    pre-quantisation values in code units, the P scale of each (row, block),
    the BLASST predicate margins (B,H,R,blocks), the per-row skipped-block
    counts and ``flip_allowance`` (B,H,R,D): the largest output change that
    one-step flips of P codes lying within 2^-15 (relative) of an E4M3
    rounding midpoint could cause -- the codes that fp32-level differences in
    evaluating the same scores (exp2, reciprocals, summation order) can flip."""
    B, H, S, D = q.shape
    dev_rows = torch.arange(S) if rows is None else torch.as_tensor(rows)
    R = dev_rows.numel()
    qf = q.float()[:, :, dev_rows]
    kf = k.float()
    vf = v.float()
    sm = _f32(sm_scale)

    p_kind = {"elementwise": 0, "mx": 1, "dynamic": 2}[p_quant_mode]
    use_blasst = blasst_lambda is not None
    if use_blasst:
        if not (0.0 < float(blasst_lambda) < 1.0):
            raise ValueError(f"blasst_lambda must be in (0, 1); got {blasst_lambda}")
        log_lam = math.log(float(blasst_lambda))
        fill_kind, fill_alpha, uta_bins = parse_blasst_fill(blasst_fill_mode, alpha=blasst_fill_alpha,
                                                            uta_bins=blasst_uta_bins)
        if fill_kind == FILL_UTA and block_n % uta_bins:
            raise ValueError(f"blasst UTA bins ({uta_bins}) must divide block_n ({block_n})")
    has_qm = qm is not None
    if has_qm:
        qm_rows = qm.permute(0, 2, 1, 3).float()[:, :, dev_rows // q_smooth_block]   # (B,H,R,D)
        ks = k_smooth.float()
    if rowmax_est is not None:
        rme = rowmax_est.float()[:, :, dev_rows]
        m_i = rme.clone()
    elif rowmax_init is not None:
        rme = rowmax_init.float()[:, :, dev_rows]
        m_i = rme.clone()
    else:
        rme = torch.zeros(B, H, R)
        m_i = torch.full((B, H, R), -math.inf)
    l_i = torch.zeros(B, H, R)
    acc = torch.zeros(B, H, R, D)
    c_acc = torch.zeros(B, H, R, D)
    max_seen = torch.full((B, H, R), -math.inf)
    skipped = torch.zeros(B, H, R)
    total = torch.zeros(B, H, R)
    row_valid = (dev_rows < S).float()
    dbg = {"skip": [], "codes": [], "x": [], "sP": [], "s": [], "margin": []} if return_debug else None
    if dbg is not None:
        # output change that one-step flips of rounding-edge P codes could cause
        alw = torch.zeros(B, H, R, D)
        alw_c = torch.zeros(B, H, R, D)
    if scores_log2 is not None:
        scores_log2 = scores_log2.float()
        if scores_log2.shape != (B, H, R, S):
            raise ValueError(f"scores_log2 must be {(B, H, R, S)}; got {tuple(scores_log2.shape)}")

    for start_n in range(0, S, block_n):
        n1 = min(start_n + block_n, S)
        nb = n1 - start_n
        col_mask = torch.zeros(block_n, dtype=torch.bool)
        col_mask[:nb] = True
        kb = torch.zeros(B, H, block_n, D)
        kb[:, :, :nb] = kf[:, :, start_n:n1]
        vb = torch.zeros(B, H, block_n, D)
        vb[:, :, :nb] = vf[:, :, start_n:n1]
        if scores_log2 is None:
            s = torch.matmul(qf, kb.transpose(-2, -1)) * sm
            if has_qm:
                ksb = torch.zeros(B, H, block_n, D)
                ksb[:, :, :nb] = ks[:, :, start_n:n1]
                corr = torch.matmul(qm_rows, ksb.transpose(-2, -1)) * sm
                s = s + corr
        else:
            s = torch.zeros(B, H, R, block_n)
            s[..., :nb] = scores_log2[..., start_n:n1] / _f32(LOG2E)
        s = torch.where(col_mask, s, torch.tensor(-math.inf))

        skip = torch.zeros(B, H, R, dtype=torch.bool)
        if use_blasst:
            block_max = s.amax(-1)
            m_ij = torch.maximum(m_i, block_max)
            skip = (block_max - m_ij) < log_lam
            alpha = torch.exp2((m_i - m_ij) * LOG2E)
            alpha = torch.where(skip, torch.ones_like(alpha), alpha)
            m_ij = torch.where(skip, m_i, m_ij)
            skipped += skip.float()
            total += row_valid
            if dbg is not None:
                # distance of the skip predicate from its threshold (skip iff < 0)
                dbg["margin"].append((block_max - torch.maximum(m_i, block_max)) - log_lam)
        elif rowmax_est is not None:
            if p_kind == 2:
                block_max = s.amax(-1)
                max_seen_ij = torch.maximum(max_seen, block_max)
                up_t = 16.0 / LOG2E
                down_t = 32.0 / LOG2E
                under = (block_max - m_i) > up_t
                over = (m_i - max_seen_ij) > down_t
                adjust = under | over
                down_b = torch.maximum(max_seen_ij + down_t, m_i - 80.0)
                down_m = torch.where(l_i == 0.0, max_seen_ij, down_b)
                adj_m = torch.where(under, block_max, down_m)
                m_ij = torch.where(adjust, adj_m, m_i)
                alpha_u = torch.exp2((m_i - m_ij) * LOG2E)
                alpha_u = torch.where(l_i == 0.0, torch.zeros_like(alpha_u), alpha_u)
                alpha = torch.where(adjust, alpha_u, torch.ones_like(alpha_u))
                max_seen = max_seen_ij
            else:
                m_ij = rme
                alpha = torch.ones(B, H, R)
        else:
            m_ij = torch.maximum(m_i, s.amax(-1))
            alpha = torch.exp2((m_i - m_ij) * LOG2E)

        if p_kind == 0:
            z = (s - m_ij[..., None]) * LOG2E + float(p_max_offset)
        else:
            z = (s - m_ij[..., None]) * LOG2E
        p = torch.exp2(z)
        p = torch.where(col_mask, p, torch.zeros_like(p))

        if use_blasst:
            if fill_kind == FILL_ZERO:
                p = torch.where(skip[..., None], torch.zeros_like(p), p)
            else:
                p_exact = torch.where(skip[..., None], torch.zeros_like(p), p)
                safe_n = float(max(nb, 1))
                fill_offset = float(p_max_offset) if p_kind == 0 else 0.0
                s_stat = torch.where(col_mask, s, torch.zeros_like(s))
                mean = s_stat.sum(-1) / safe_n
                max_bound = safe_n * torch.exp2((block_max - m_ij) * LOG2E + fill_offset)
                p_fill = torch.zeros_like(p)
                sel = skip[..., None] & col_mask
                if fill_kind == FILL_MAX:
                    fill_p = max_bound * fill_alpha / safe_n
                    p_fill = torch.where(sel, fill_p[..., None], p_fill)
                elif fill_kind == FILL_MEAN:
                    mass = fill_alpha * safe_n * torch.exp2((mean - m_ij) * LOG2E + fill_offset)
                    mass = torch.minimum(mass, max_bound)
                    p_fill = torch.where(sel, (mass / safe_n)[..., None], p_fill)
                elif fill_kind == FILL_LOGN:
                    centered = torch.where(col_mask, s - mean[..., None], torch.zeros_like(s))
                    var = (centered * centered).sum(-1) / safe_n
                    mass = safe_n * torch.exp2((mean + 0.5 * var - m_ij) * LOG2E + fill_offset)
                    mass = torch.minimum(mass, max_bound)
                    p_fill = torch.where(sel, (mass / safe_n)[..., None], p_fill)
                elif fill_kind == FILL_SAMPLE8:
                    stride = block_n // 8 if block_n >= 8 else 1
                    rel = torch.arange(block_n)
                    smask = ((rel % stride) == 0) & col_mask
                    cnt = float(max(int(smask.sum()), 1))
                    sp = torch.exp2((s - m_ij[..., None]) * LOG2E + fill_offset)
                    sp = torch.where(smask, sp, torch.zeros_like(sp))
                    mass = fill_alpha * safe_n * sp.sum(-1) / cnt
                    mass = torch.minimum(mass, max_bound)
                    p_fill = torch.where(sel, (mass / safe_n)[..., None], p_fill)
                elif fill_kind == FILL_THR:
                    off_scale = 2.0 ** float(p_max_offset) if p_kind == 0 else 1.0
                    mass = fill_alpha * safe_n * float(blasst_lambda) * off_scale
                    p_fill = torch.where(sel, torch.full_like(p, mass / safe_n), p_fill)
                else:
                    rel = torch.arange(block_n)
                    bsz = block_n // uta_bins
                    for bi in range(uta_bins):
                        bmask = (rel >= bi * bsz) & (rel < (bi + 1) * bsz) & col_mask
                        bc = float(max(int(bmask.sum()), 1))
                        bmean = torch.where(bmask, s, torch.zeros_like(s)).sum(-1) / bc
                        bmax = torch.where(bmask, s, torch.full_like(s, -math.inf)).amax(-1)
                        bound = bc * torch.exp2((bmax - m_ij) * LOG2E + fill_offset)
                        mass = fill_alpha * bc * torch.exp2((bmean - m_ij) * LOG2E + fill_offset)
                        mass = torch.minimum(mass, bound)
                        p_fill = torch.where(skip[..., None] & bmask, (mass / bc)[..., None], p_fill)
                p = p_exact + p_fill
            if dbg is not None:
                dbg["skip"].append(skip.clone())

        l_i = l_i * alpha + p.sum(-1)

        # x: P in code units; codes = e4m3(x) (saturating); p_deq = bf16(code * s_P)
        if p_kind == 0:
            sP = torch.ones(B, H, R)
            x = p
        elif p_kind == 1:
            ra = p.abs().amax(-1).clamp_min(float(np.float32(1e-4)))
            e = np.clip(ceil_log2_exact((ra / _f32(FP8_MAX)).numpy()), -127, 127)
            sP = torch.from_numpy(np.ldexp(np.float32(1.0), e).astype(np.float32))
            x = torch.clamp(p / sP[..., None], -FP8_MAX, FP8_MAX)
        else:
            ra = p.abs().amax(-1).clamp_min(float(np.float32(1e-12)))
            sP = ra / _f32(FP8_MAX)
            x = torch.clamp(p / sP[..., None], -FP8_MAX, FP8_MAX)
        codes = torch.from_numpy(fp8.encode(x.contiguous().numpy()))
        if force_codes is not None:
            fc, fm = force_codes
            codes[..., :nb] = torch.where(fm[..., start_n:n1], fc[..., start_n:n1], codes[..., :nb])
        vals = torch.from_numpy(fp8.decode(codes.numpy()))
        if p_kind == 0:
            p_deq = vals.to(torch.bfloat16).float()
        else:
            p_deq = (vals * sP[..., None]).to(torch.bfloat16).float()
        if dbg is not None:
            edge = rounding_edge_step(x)
            if p_kind == 1:
                # an MX exponent at a power-of-two edge re-rounds every code of the block
                lr = np.log2((ra / _f32(FP8_MAX)).double().numpy())
                e_edge = torch.from_numpy(np.abs(lr - np.round(lr)) <= EDGE_REL)
                step_all = 2.0 * rounding_edge_step(x, rel=1.0)
                edge = torch.where(e_edge[..., None], step_all, edge)
            w = torch.where(col_mask, edge * sP[..., None], torch.zeros_like(edge))
            dpv = torch.matmul(w, vb.abs())
            if v_block_scale is not None:
                dpv = dpv * v_block_scale.float()[:, start_n // v_block_size, :].abs()[..., None, None]
            alw = alw * alpha[..., None] + dpv
            if v_alpha is not None:
                alw_c = alw_c * alpha[..., None] + w.sum(-1)[..., None] * v_alpha.float()[
                    :, start_n // v_smooth_block].abs()[:, :, None, :]
            dbg["s"].append(s[..., :nb].clone())
            dbg["codes"].append(codes[..., :nb].clone())
            dbg["x"].append(x[..., :nb].clone())
            dbg["sP"].append(sP.clone())

        pv = torch.matmul(p_deq, vb)
        if v_block_scale is not None:
            svb = v_block_scale.float()[:, start_n // v_block_size, :]     # (B, H)
            pv = pv * svb[..., None, None]
        acc = acc * alpha[..., None] + pv
        if v_alpha is not None:
            av = v_alpha.float()[:, start_n // v_smooth_block]             # (B, H, D)
            rs = p_deq.sum(-1)
            c_acc = c_acc * alpha[..., None] + rs[..., None] * av[:, :, None, :]
        m_i = m_ij

    inv_l = 1.0 / l_i[..., None]
    out_main = acc if v_block_scale is not None else acc * v_scale.float()[:, :, None, :]
    out = (out_main + c_acc) * inv_l if v_alpha is not None else out_main * inv_l
    out = out.to(torch.bfloat16)
    result = [out]
    if return_blasst_stats:
        nblk = (S + block_m - 1) // block_m
        st = torch.zeros(nblk, B * H, 2)
        blk = dev_rows // block_m
        sk = skipped.reshape(B * H, R)
        tt = total.reshape(B * H, R)
        for bi in range(nblk):
            sel = blk == bi
            st[bi, :, 0] = sk[:, sel].sum(-1)
            st[bi, :, 1] = tt[:, sel].sum(-1)
        result.append(st)
    if dbg is not None:
        dbg["codes"] = torch.cat(dbg["codes"], -1)
        dbg["x"] = torch.cat(dbg["x"], -1)
        dbg["sP"] = torch.stack(dbg["sP"], -1)
        dbg["s"] = torch.cat(dbg["s"], -1)
        dbg["margin"] = torch.stack(dbg["margin"], -1) if dbg["margin"] else None
        dbg["row_skips"] = skipped
        scale_main = 1.0 if v_block_scale is not None else v_scale.float().abs()[:, :, None, :]
        dbg["flip_allowance"] = (alw * scale_main + alw_c) / l_i[..., None].abs()
        result.append(dbg)
    return result[0] if len(result) == 1 else tuple(result)
