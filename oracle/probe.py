"""CPU restatement of the diagnostic probes (test infrastructure only).

* ``p_requant_rows`` -- reference ``p_requant.py:12-41`` (kernel) / ``:44-73``
  (wrapper): per row p = e4m3(2^((x - max) * (sm_scale * log2 e) +
  p_max_offset)), row_sum = sum p, lse = max * sm_scale + ln(row_sum) -
  p_max_offset * ln 2.  The scale constant is folded in double and rounded
  to fp32 once, as the reference's constexpr product is; z is one fp32
  rounding of (x - max) * c + offset.
* ``rowmax_counts`` -- reference ``bench/count_rowmax_updates_triton.py:
  100-171`` (the K-loop update rules and the six counters), over a given
  score matrix, in natural units (the reference) or log2 units (the HIP
  kernel).
* ``reference_scores`` -- the scores that diagnostic sees (``:128-139``,
  driver ``:228-245``): bf16 dequantised Q/K of the preprocessed operands,
  ``q . k * sm_scale + (qm . K_smooth) * sm_scale``, and the qm_k estimate.
* ``kernel_scores_log2`` -- the same scores as the HIP counter kernel forms
  them from FP8 codes: ``(q_codes . k_codes) * (sm_scale log2e * sq * sk) +
  bias`` in log2 units.

Pinned by ``tests/test_oracle_probe.py``: p_requant_rows against float64
softmax / logsumexp and the exact code of 2^offset (and saturation);
rowmax_counts on hand-built tile sequences whose counts follow from the
rules by hand, and unit invariance (natural vs log2 units).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import fp8
from . import pipeline as opipe
from . import quant as oq

LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453
COUNTER_NAMES = ("updates", "rescales", "upward_updates", "downward_updates", "rows_with_update",
                 "max_updates_per_row")


def p_requant_rows(scores: torch.Tensor, *, sm_scale: float, p_max_offset: int = 8):
    """(codes uint8 (B,M,N), row_sum fp32 (B,M), lse fp32 (B,M)) of CPU ``scores``."""
    x = scores.float()
    mx = x.amax(dim=-1, keepdim=True)
    c = np.float32(float(sm_scale) * LOG2E)
    d = (x - mx).double()
    # one rounding of d * c + offset: the double product of two fp32 values is exact
    z = (d * float(c) + float(p_max_offset)).float()
    p = torch.exp2(z)
    codes = torch.from_numpy(fp8.encode(p.numpy()))
    row_sum = p.double().sum(dim=-1).float()
    lse = (mx.squeeze(-1).double() * float(np.float32(sm_scale)) + torch.log(row_sum.double())).float() \
        - np.float32(p_max_offset * LN2)
    return codes, row_sum, lse.float()


def rowmax_counts(scores: torch.Tensor, m0: torch.Tensor | None, *, up: float, down: float, use_estimate: bool,
                  down_always: bool = False, mass_floor: float = 1e-6, block_n: int = 64,
                  units: str = "natural") -> dict:
    """The six counters over rows of ``scores`` (R, N) fp32.

    ``units="natural"``: scores are natural-log logits (the reference); the
    thresholds (log2 units) become ``up / log2 e`` and p = 2^((s - m) log2 e).
    ``units="log2"``: scores are in log2 units (the HIP kernel); thresholds
    are used as given, the ``m - 80`` bound becomes ``m - 80 log2 e``.
    ``m0``: (R,) initial row max of the estimated mode.
    """
    s = scores.float()
    r, n = s.shape
    if units == "natural":
        up_t = torch.tensor(up / LOG2E, dtype=torch.float32)
        down_t = torch.tensor(down / LOG2E, dtype=torch.float32)
        shift = torch.tensor(80.0, dtype=torch.float32)
        to2 = torch.tensor(LOG2E, dtype=torch.float32)
    elif units == "log2":
        up_t = torch.tensor(up, dtype=torch.float32)
        down_t = torch.tensor(down, dtype=torch.float32)
        shift = torch.tensor(80.0 * LOG2E, dtype=torch.float32)
        to2 = None
    else:
        raise ValueError(units)
    m = m0.float().clone() if use_estimate else torch.full((r,), -math.inf)
    l = torch.zeros(r)
    seen = torch.full((r,), -math.inf)
    count = torch.zeros(r, dtype=torch.int64)
    tot = dict.fromkeys(COUNTER_NAMES[:4], 0)
    for j0 in range(0, n, block_n):
        t = s[:, j0:j0 + block_n]
        bmax = t.amax(dim=1)
        if use_estimate:
            seen_ij = torch.maximum(seen, bmax)
            under = (bmax - m) > up_t
            over = (m - seen_ij) > down_t
            if not down_always:
                over = over & (l < mass_floor)
            adjust = under | over
            down_bounded = torch.maximum(seen_ij + down_t, m - shift)
            down_m = torch.where(l == 0.0, seen_ij, down_bounded)
            m_new = torch.where(adjust, torch.where(under, bmax, down_m), m)
            diff = m - m_new
            a_up = torch.exp2(diff * to2 if to2 is not None else diff)
            a_up = torch.where(l == 0.0, torch.zeros_like(a_up), a_up)
            alpha = torch.where(adjust, a_up, torch.ones_like(a_up))
            seen = seen_ij
            rescale = adjust & (l != 0.0)
            tot["upward_updates"] += int((adjust & under).sum())
            tot["downward_updates"] += int((adjust & ~under).sum())
        else:
            first = m == -math.inf
            adjust = first | ((bmax - m) > up_t)
            m_new = torch.where(adjust, bmax, m)
            diff = m - m_new
            alpha = torch.exp2(diff * to2 if to2 is not None else diff)
            alpha = torch.where(first, torch.zeros_like(alpha), alpha)
            rescale = adjust & ~first
            tot["upward_updates"] += int(adjust.sum())
        e = t - m_new[:, None]
        p_sum = torch.exp2(e * to2 if to2 is not None else e).sum(dim=1)
        l = l * alpha + p_sum
        m = m_new
        tot["updates"] += int(adjust.sum())
        tot["rescales"] += int(rescale.sum())
        count += adjust.long()
    tot["rows_with_update"] = int((count > 0).sum())
    tot["max_updates_per_row"] = int(count.max()) if r else 0
    return tot


def reference_scores(q, k, v, cfg, *, sm_scale=None):
    """(scores (B*H*S, S) fp32 natural units, estimate (B*H*S,)) of the reference
    diagnostic on NHD CPU q/k/v (S already padded)."""
    b, s, h, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    q_work, k_work, _, qm, _, _, _ = opipe.preprocess(q, k, v, cfg)
    qc, qs, qmeta = opipe.quant_qk(q_work, cfg)
    kc, ks, kmeta = opipe.quant_qk(k_work, cfg)
    q_deq = opipe.dequant_qk(qc, qs, qmeta, torch.bfloat16).permute(0, 2, 1, 3).float()
    k_deq = opipe.dequant_qk(kc, ks, kmeta, torch.bfloat16).permute(0, 2, 1, 3).float()
    sm = torch.tensor(sm_scale, dtype=torch.float32)
    sc = torch.matmul(q_deq, k_deq.transpose(-1, -2)) * sm
    k_s = k_work.to(torch.bfloat16).permute(0, 2, 1, 3).float()            # (B,H,S,D)
    qm_b = qm.permute(0, 2, 1, 3).float()                                    # (B,H,G,D)
    corr = torch.matmul(qm_b, k_s.transpose(-1, -2)) * sm                    # (B,H,G,S)
    corr = corr.repeat_interleave(cfg.q_smooth_block_size, dim=2)
    sc = sc + corr
    from . import attention as oattn
    est = oattn.estimate_rowmax_qm_k(qm, k_work, block_q=cfg.q_smooth_block_size, sm_scale=sm_scale)
    return sc.reshape(b * h * s, s), est.reshape(b * h * s)


def kernel_scores_log2(q_codes, q_scale, k_codes, k_scale, bias, rowmax, *, s, qk_block, q_group, sm_scale):
    """(scores (B*H*S, S) fp32 log2 units, estimate (B*H*S,)) as the HIP counter
    kernel forms them; codes (B,H,P,D) uint8, fp8_block scales (B,H,nblk),
    bias (B,H,G,P), rowmax (B,H,G) -- all CPU tensors."""
    b, h, _, d = q_codes.shape
    qd = oq.decode(q_codes[:, :, :s].contiguous()).double()
    kd = oq.decode(k_codes[:, :, :s].contiguous()).double()
    dot = torch.matmul(qd, kd.transpose(-1, -2)).float()                     # MFMA result
    sml2 = np.float32(float(np.float32(sm_scale)) * LOG2E)   # the kernel receives sm_scale as fp32
    rows = torch.arange(s)
    qC = (torch.tensor(sml2) * q_scale[:, :, rows // qk_block].float())      # fp32 product
    C = qC[..., :, None] * k_scale[:, :, rows // qk_block].float()[..., None, :]
    g = (rows // q_group).clamp(max=bias.shape[2] - 1)
    bb = bias[:, :, g, :s].float()                                            # (B,H,S,S)
    u = (dot.double() * C.double() + bb.double()).float()                    # one rounding: fmaf
    est = rowmax[:, :, g].float()
    return u.reshape(b * h * s, s), est.reshape(b * h * s)
