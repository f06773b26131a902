"""Row-max update / rescale counters of the dynamic-P K loop.

MI355X counterpart of the reference diagnostic
``bench/count_rowmax_updates_triton.py`` (kernel ``:27-171``, driver
``:196-334``), whose counts the reference README reports (``README.md:111-
139``).  For each query row the K loop visits 64-key tiles and applies one of
two coordinate rules:

* ``fa4_online``: the row max starts at -inf; a tile updates it when
  ``tile_max - m > up`` (the first tile always does); every update after the
  first is a rescale;
* ``estimated``: the row max starts at the qm_k estimate; a tile moves it up
  to the tile max when ``tile_max - m > up``, or down when
  ``m - max_seen > down`` (and, unless ``down_always``, the row's mass
  ``l < mass_floor``), to ``max_seen`` while ``l == 0`` and otherwise to
  ``max(max_seen + down, m - 80 / ln 2)``; an update with ``l != 0`` is a
  rescale.

Thresholds are in log2 units, as in the reference driver.  The counts come
from ``lbfq_rowmax_count``, one HIP kernel over the same FP8 codes, scales,
qm correction table and row-max estimate the attention kernel reads.

Command line (same arguments as the reference driver)::

    python -m low_bit_fake_quant.rowmax_counters --workload call.pt --output out.json
"""

from __future__ import annotations

import argparse
import json
import math
from pathlib import Path
from typing import Iterable, Optional

import torch

from . import _lib
from .attention import QuantizedOperands, _lazy_preprocess, quantize_operands
from .config import QuantConfig

COUNTER_NAMES = ("updates", "rescales", "upward_updates", "downward_updates", "rows_with_update",
                 "max_updates_per_row")
BLOCK_N = 64
MASS_FLOOR = 1.0e-6


def counter_config(*, q_smooth_block: int = 256, q_kmeans_k: Optional[int] = 32, fp8_block_size: int = 64,
                   block_m: int = 64, block_n: int = BLOCK_N) -> QuantConfig:
    """The configuration the reference driver builds (``:213-227``)."""
    return QuantConfig(qk_quant="fp8_block", v_quant="fp8_channel", smoothing="full", q_kmeans_k=q_kmeans_k,
                       q_smooth_block_size=q_smooth_block, fp8_block_size=fp8_block_size, v_smooth_mode="off",
                       v_kmeans_k=None, p_quant="dynamic", rowmax_mode="qm_k", p_requant=True,
                       p_requant_block_m=block_m, p_requant_block_n=block_n)


def count_rowmax_updates(ops: QuantizedOperands, cfg: QuantConfig, *, sm_scale: float, up_threshold: float,
                         down_threshold: float, use_estimate: bool, down_always: bool = False,
                         mass_floor: float = MASS_FLOOR) -> dict:
    """The six counters over all rows of the quantised operands."""
    if cfg.qk_quant != "fp8_block":
        raise ValueError("rowmax counters need qk_quant='fp8_block'")
    if cfg.p_requant_block_n != BLOCK_N:
        raise ValueError(f"rowmax counters use {BLOCK_N}-key tiles; got block_n={cfg.p_requant_block_n}")
    if use_estimate and ops.rowmax is None:
        raise ValueError("the estimated mode needs the qm_k row-max estimate (rowmax_mode='qm_k')")
    dev = ops.q_codes.device
    counters = torch.zeros(6, dtype=torch.int64, device=dev)
    p = _lib.RowmaxCountParams()
    p.B, p.H, p.S, p.D, p.s_pitch = ops.b, ops.h, ops.s, ops.d, ops.P
    p.q_codes, p.k_codes = ops.q_codes.data_ptr(), ops.k_codes.data_ptr()
    p.q_scale, p.k_scale = ops.q_scale.data_ptr(), ops.k_scale.data_ptr()
    p.qk_block = int(cfg.fp8_block_size)
    p.bias = _lib.ptr(ops.bias)
    p.rowmax_est = _lib.ptr(ops.rowmax)
    p.q_group = int(cfg.q_smooth_block_size) if ops.bias is not None else 0
    p.sm_scale = float(sm_scale)
    p.up_threshold_log2, p.down_threshold_log2 = float(up_threshold), float(down_threshold)
    p.mass_floor = float(mass_floor)
    p.down_always, p.use_estimate = int(bool(down_always)), int(bool(use_estimate))
    p.counters = counters.data_ptr()
    lib = _lib.load()
    _lib.check(lib.lbfq_rowmax_count(p, _lib.stream_handle(dev)), "rowmax_count")
    vals = counters.cpu().tolist()
    return dict(zip(COUNTER_NAMES, vals))


def _with_rates(c: dict, rows: int, row_tiles: int) -> dict:
    out = dict(c)
    out["updates_per_row_avg"] = c["updates"] / rows
    out["rescales_per_row_avg"] = c["rescales"] / rows
    out["update_rate_per_row_tile"] = c["updates"] / row_tiles
    out["rescale_rate_per_row_tile"] = c["rescales"] / row_tiles
    return out


def threshold_pairs(thresholds: Iterable[float], up: Optional[Iterable[float]] = None,
                    down: Optional[Iterable[float]] = None) -> list:
    """(up, down) pairs as the reference driver forms them (``:248-254``)."""
    if up is not None or down is not None:
        ups = list(up) if up is not None else list(thresholds)
        downs = list(down) if down is not None else list(thresholds)
        return [(float(u), float(d)) for u in ups for d in downs]
    return [(float(t), float(t)) for t in thresholds]


def rowmax_update_report(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cfg: QuantConfig, *,
                         pairs: Iterable[tuple], down_always: bool = False,
                         sm_scale: Optional[float] = None) -> dict:
    """Counters for every (up, down) pair and both rules, with per-row rates.

    q/k/v are NHD on the GPU with S a multiple of the block sizes.
    """
    b, s, h, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    prep = _lazy_preprocess(q, k, v, cfg)
    ops = quantize_operands(prep, cfg, sm_scale)
    rows = b * h * s
    row_tiles = rows * ((s + BLOCK_N - 1) // BLOCK_N)
    results = {}
    for up, down in pairs:
        key = f"up{up}_down{down}"
        results[key] = {}
        for name, est in (("fa4_online", False), ("estimated", True)):
            c = count_rowmax_updates(ops, cfg, sm_scale=sm_scale, up_threshold=up, down_threshold=down,
                                     use_estimate=est, down_always=down_always)
            results[key][name] = _with_rates(c, rows, row_tiles)
    return results


def _pad_to(q, k, v, block: int):
    pad = (block - q.shape[1] % block) % block
    if pad == 0:
        return q, k, v, 0
    b, _, h, d = q.shape
    return (torch.cat([q, q.new_zeros(b, pad, h, d)], dim=1),
            torch.cat([k, k[:, -1:].expand(b, pad, h, d)], dim=1),
            torch.cat([v, v[:, -1:].expand(b, pad, h, d)], dim=1), pad)


def main(argv=None) -> dict:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--workload", type=Path, required=True, help="dump with CPU tensors query/key/value")
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--q-smooth-block", type=int, default=256)
    ap.add_argument("--q-kmeans-k", type=int, default=32)
    ap.add_argument("--fp8-block-size", type=int, default=64)
    ap.add_argument("--block-m", type=int, default=64)
    ap.add_argument("--block-n", type=int, default=BLOCK_N)
    ap.add_argument("--thresholds", nargs="+", type=float, default=[8.0, 16.0])
    ap.add_argument("--up-thresholds", nargs="+", type=float, default=None)
    ap.add_argument("--down-thresholds", nargs="+", type=float, default=None)
    ap.add_argument("--down-always", action="store_true")
    args = ap.parse_args(argv)

    from .wan_hook import load_qkv_dump
    device = torch.device(args.device)
    q, k, v = load_qkv_dump(args.workload, device=device)
    orig_s = q.shape[1]
    q, k, v, pad = _pad_to(q, k, v, args.q_smooth_block)
    cfg = counter_config(q_smooth_block=args.q_smooth_block, q_kmeans_k=args.q_kmeans_k,
                         fp8_block_size=args.fp8_block_size, block_m=args.block_m, block_n=args.block_n)
    pairs = threshold_pairs(args.thresholds, args.up_thresholds, args.down_thresholds)
    results = rowmax_update_report(q, k, v, cfg, pairs=pairs, down_always=args.down_always)
    b, s, h, d = q.shape
    report = {
        "workload": str(args.workload), "shape": [b, s, h, d], "orig_s": orig_s, "pad": pad,
        "q_smooth_block": args.q_smooth_block, "q_kmeans_k": args.q_kmeans_k,
        "fp8_block_size": args.fp8_block_size, "block_m": args.block_m, "block_n": args.block_n,
        "results": results, "down_always": args.down_always,
    }
    args.output.parent.mkdir(parents=True, exist_ok=True)
    args.output.write_text(json.dumps(report, indent=2))
    print(json.dumps(report, indent=2))
    return report


if __name__ == "__main__":
    main()
