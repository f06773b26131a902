"""CPU restatement of the BLASST tile-skip simulator (test infrastructure only).

Follows ``simulate_workload`` of the reference ``blasst_skip.py:389-654``
tile by tile on the CPU in fp32:

* per-head static FP8 quant (``:278-297``): scale = max(amax / 448, FLT_MIN)
  over each head's (S, D) slab, deq = e4m3(x / scale) * scale, then the matmul
  operand is deq rounded to the matmul dtype;
* per 128-row tile: scores = (q . k) * sm_scale (fp32), block maxima over 128
  keys, running max = cumulative max, final max (``:497-506``);
* rungs: exact softmax (``:484-491``), online weights exp(s - rm) *
  exp(rm - M) (``:508-519``), static P e4m3(exp(s - rm) * 256) / 256 scaled by
  exp(rm - M) with the unquantised denominator (``:521-570``); P rounded to the
  matmul dtype before PV, fp32 accumulation;
* tile predicate: max over the tile's rows of (bmax - rm) >= log(threshold),
  empty-tile safeguard = first block of largest max-over-rows bmax
  (``:584-619``); dropped mass = sum over dropped blocks of the block's share
  of the unquantised row mass.

Pinned by ``tests/test_oracle_blasst_sim.py``: the exact rung against float64
softmax attention; the online rung against float64 softmax over the
dequantised operands; skip at threshold 0 equals the static rung bitwise;
skip rate monotone in the threshold on a workload built to be skippable; the
safeguard fires at threshold 1; the per-tile keep masks against a brute-force
per-row evaluation of the predicate; the E4M3 fake quant against
``torch.float8_e4m3fn``.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import fp8

TILE = 128
FLT_MIN = float(np.finfo(np.float32).tiny)


def _e4m3_rt(x: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(fp8.decode(fp8.encode(x.contiguous().numpy()))).float()


def _to_mm(x: torch.Tensor, mm_dtype) -> torch.Tensor:
    return x.to(mm_dtype).float()


def head_quant(x3: torch.Tensor):
    """(deq fp32 (S,H,D), scale (H,), stats dict) of an (S, H, D) tensor."""
    xf = x3.float()
    amax = xf.abs().amax(dim=(0, 2))
    scale = torch.clamp(amax / torch.tensor(448.0), min=FLT_MIN)
    scaled = xf / scale.view(1, -1, 1)
    q = _e4m3_rt(scaled)
    deq = q * scale.view(1, -1, 1)
    n = xf.numel()
    stats = {"saturation_rate": int((scaled.abs() > 448.0).sum()) / n,
             "underflow_zero_rate": int(((q == 0) & (scaled != 0)).sum()) / n,
             "roundtrip_rmse": math.sqrt(float(((deq.double() - xf.double()) ** 2).sum()) / n)}
    return deq, scale, stats


def _tile_stats(qh, kh, sm, rows):
    """scores (H, m, S), block max (H, m, nb), running max, final max for one tile."""
    sc = torch.matmul(qh[:, rows], kh.transpose(1, 2)) * torch.tensor(sm, dtype=torch.float32)
    h, m, s = sc.shape
    bmax = sc.view(h, m, s // TILE, TILE).amax(-1)
    rm = torch.cummax(bmax, dim=-1).values
    return sc, bmax, rm, rm[..., -1]


def simulate(q, k, v, *, skip_thresholds=(), mm_dtype=torch.bfloat16):
    """dict with 'bf16_ref', 'fp8_qkv', 'fp8_static_p' (S,H,D) outputs, 'skip'
    {th: (S,H,D)}, 'skip_rate' {th}, 'force' {th}, 'dropped' {th: (H,S)},
    'keep' {th: (H, nM, nb) bool}, 'stats' {q,k,v,p}.  q/k/v: (1,S,H,D) CPU."""
    _, s, h, d = q.shape
    sm = 1.0 / math.sqrt(d)
    nb = s // TILE
    heads = lambda t: t.permute(1, 0, 2).contiguous()  # (S,H,D) -> (H,S,D)
    qr, kr, vr = (heads(_to_mm(t[0], mm_dtype)) for t in (q, k, v))
    deqs, stats = [], {}
    for name, t in (("q", q), ("k", k), ("v", v)):
        dq, _, st = head_quant(t[0])
        deqs.append(heads(_to_mm(dq, mm_dtype)))
        stats[name] = st
    qd, kd, vd = deqs
    rnd = (lambda x: x.to(torch.bfloat16).float()) if mm_dtype == torch.bfloat16 else (lambda x: x)
    ths = list(skip_thresholds)
    res = {k_: torch.empty(s, h, d) for k_ in ("bf16_ref", "fp8_qkv", "fp8_static_p")}
    res.update(skip={th: torch.empty(s, h, d) for th in ths}, dropped={th: torch.empty(h, s) for th in ths},
               keep={th: torch.empty(h, s // TILE, nb, dtype=torch.bool) for th in ths},
               skip_rate={th: 0 for th in ths}, force={th: 0 for th in ths})
    uf = cnt = 0
    sqe = 0.0
    for mt in range(s // TILE):
        rows = slice(mt * TILE, (mt + 1) * TILE)
        # exact rung on the unquantised operands
        sc, _, _, _ = _tile_stats(qr, kr, sm, rows)
        p = torch.exp(sc - sc.amax(-1, keepdim=True))
        res["bf16_ref"][rows] = (torch.matmul(rnd(p), vr) / p.sum(-1, keepdim=True)).permute(1, 0, 2)
        # FP8 rungs
        sc, bmax, rm, fm = _tile_stats(qd, kd, sm, rows)
        m = sc.shape[1]
        sb = sc.view(h, m, nb, TILE)
        on = torch.exp(sb - rm.unsqueeze(-1))
        resc = torch.exp(rm - fm.unsqueeze(-1)).unsqueeze(-1)
        w = on * resc
        res["fp8_qkv"][rows] = (torch.matmul(rnd(w.view(h, m, s)), vd) / w.view(h, m, s).sum(-1, keepdim=True)
                                ).permute(1, 0, 2)
        scaled = on * 256.0
        pq8 = _e4m3_rt(scaled)
        pq = pq8 / 256.0
        uf += int(((pq8 == 0) & (scaled != 0)).sum())
        cnt += on.numel()
        sqe += float(((pq.double() - on.double()) ** 2).sum())
        pw = rnd(pq * resc)                                            # (h, m, nb, TILE)
        lb = w.sum(-1)                                                 # (h, m, nb)
        vb = vd.view(h, nb, TILE, d)
        pv = torch.einsum("hmjk,hjkd->hmjd", pw, vb)                   # per-block partial sums
        res["fp8_static_p"][rows] = (pv.sum(2) / lb.sum(-1, keepdim=True).clamp_min(1e-30)).permute(1, 0, 2)
        tile_margin = (bmax - rm).amax(dim=1)                          # (h, nb)
        tile_bmax = bmax.amax(dim=1)
        for th in ths:
            lt = -math.inf if th <= 0 else math.log(th)
            keep = tile_margin >= lt
            none = ~keep.any(-1)
            if none.any():
                best = tile_bmax.argmax(-1)
                keep[none, best[none]] = True
                res["force"][th] += int(none.sum())
            res["keep"][th][:, mt] = keep
            res["skip_rate"][th] += int((~keep).sum())
            kf = keep.float()
            num = (pv * kf[:, None, :, None]).sum(2)
            den = (lb * kf[:, None, :]).sum(-1, keepdim=True).clamp_min(1e-30)
            res["skip"][th][rows] = (num / den).permute(1, 0, 2)
            frac = lb / lb.sum(-1, keepdim=True).clamp_min(1e-30)
            res["dropped"][th][:, rows] = (frac * (~keep).float()[:, None, :]).sum(-1)
    total = (s // TILE) * h * nb
    res["skip_rate"] = {th: c / total for th, c in res["skip_rate"].items()}
    stats["p"] = {"saturation_rate": 0.0, "underflow_zero_rate": uf / cnt, "roundtrip_rmse": math.sqrt(sqe / cnt)}
    res["stats"] = stats
    return res
