"""BLASST tile-skip simulator on MI355X (reference ``blasst_skip.py``).

A measurement tool beside the attention path: the FP8 fake-quant + whole-tile
BLASST skipping ablation ladder on 128-query x 128-key tiles, with per-head
static FP8 scales for Q/K/V and the static P rule ``e4m3(p * 256) / 256``.

Rungs (``LADDER``): ``bf16_ref`` (no quant, no skip), ``fp8_qkv`` (FP8 Q/K/V,
P unquantised), ``fp8_static_p`` (+ static P quant) and ``fp8_static_p_skip``
(+ the tile predicate at each skip threshold).  The skip predicate keeps key
block j of a 128-row tile iff ``max over the tile's rows of (block_max_j -
running_max_j) >= log(threshold)``, the running max being the cumulative max
of block maxima (a skipped block never raises it); a tile that keeps no block
keeps its block of largest max (``blasst_skip.py:348-386, 584-619``).

``simulate_workload`` runs on four HIP kernels (``lbfq_head_fp8_quant``,
``lbfq_blasst_scan``, ``lbfq_blasst_keep``, ``lbfq_blasst_attend``): a scan
pass forms the scores once per row and records row maxima and per-tile
margins, a keep pass turns the margins into masks, and one attend pass per
rung (per threshold for the skip rung) accumulates the output.  The tile
statistics are a few bytes per tile, so no ``S x S`` buffer exists at any
point (``guard_no_full_matrix`` keeps the reference's check for callers).

The predicate helpers (``running_row_max``, ``blasst_keep_mask``,
``blasst_tile_keep_mask``), the static P rule and the token-reorder helpers
are small tensor functions with the reference's semantics; they run wherever
their inputs live.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import _lib

E4M3_MAX = 448.0
P_STATIC_SCALE = 256.0
QUERY_TILE = 128
KEY_BLOCK = 128
DENOM_FLOOR = 1e-30

LEVEL_REFERENCE = "bf16_ref"
LEVEL_FP8_QKV = "fp8_qkv"
LEVEL_FP8_STATIC_P = "fp8_static_p"
LEVEL_FP8_SKIP = "fp8_static_p_skip"
LADDER = (LEVEL_REFERENCE, LEVEL_FP8_QKV, LEVEL_FP8_STATIC_P, LEVEL_FP8_SKIP)

MATH_BACKEND_SEQLEN_LIMIT = 8192
_STREAMING_SDPA_BACKENDS = (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION)
_ORDERED_NEG_INF = 0x007FFFFF


class FullMatrixAllocationError(RuntimeError):
    """A code path would allocate a full ``seqlen x seqlen`` buffer."""


def guard_no_full_matrix(shape, seqlen: int) -> None:
    """Raise if ``shape`` has two dimensions of at least ``seqlen``."""
    if sum(1 for d in shape if int(d) >= seqlen) >= 2:
        raise FullMatrixAllocationError(
            f"refusing to allocate full {seqlen}x{seqlen} matrix; got shape {tuple(int(d) for d in shape)}")


def select_sdpa_backends(seqlen: int, *, force_math_backend: bool, allow_math_fallback: bool):
    """Streaming SDPA backends, plus math only below ``MATH_BACKEND_SEQLEN_LIMIT``."""
    if force_math_backend:
        if seqlen >= MATH_BACKEND_SEQLEN_LIMIT:
            raise FullMatrixAllocationError(
                f"forcing the math SDPA backend at seqlen {seqlen} would materialize a "
                f"{seqlen}x{seqlen} scores matrix and OOM; refusing")
        return [SDPBackend.MATH]
    backends = list(_STREAMING_SDPA_BACKENDS)
    if allow_math_fallback and seqlen < MATH_BACKEND_SEQLEN_LIMIT:
        backends.append(SDPBackend.MATH)
    return backends


def sdpa_ground_truth(q, k, v, *, sm_scale: Optional[float] = None, allow_math_fallback: bool = False,
                      force_math_backend: bool = False) -> torch.Tensor:
    """torch SDPA of (B, S, H, D) tensors with a pinned backend set.

    The math backend, when selected, runs on float32 copies (its batched
    products in bf16 are avoided) and the result is cast back.
    """
    if q.ndim != 4:
        raise ValueError(f"q/k/v must be (B, S, H, D); got {tuple(q.shape)}")
    backends = select_sdpa_backends(q.shape[1], force_math_backend=force_math_backend,
                                    allow_math_fallback=allow_math_fallback)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    cast = force_math_backend and q.dtype != torch.float32
    qb, kb, vb = ((t.float() if cast else t).permute(0, 2, 1, 3).contiguous() for t in (q, k, v))
    with sdpa_kernel(backends):
        o = F.scaled_dot_product_attention(qb, kb, vb, scale=sm_scale)
    o = o.permute(0, 2, 1, 3).contiguous()
    return o.to(q.dtype) if cast else o


# ---- token reorder helpers (blasst_skip.py:152-262) -------------------------------

AXES = ("t", "h", "w")


def choose_local_block(t: int, h: int, w: int, tile: int = QUERY_TILE) -> tuple:
    """(bt, bh, bw) with bt*bh*bw == tile dividing (t, h, w): repeatedly double
    the side of the axis with the most blocks left, among axes that still halve."""
    if tile & (tile - 1):
        raise ValueError("tile must be a power of two")
    dims = {"t": t, "h": h, "w": w}
    blk = {"t": 1, "h": 1, "w": 1}
    while blk["t"] * blk["h"] * blk["w"] < tile:
        cand = [a for a in AXES if dims[a] // blk[a] > 1 and (dims[a] // blk[a]) % 2 == 0]
        if not cand:
            raise ValueError(f"cannot tile ({t},{h},{w}) into a {tile}-token block")
        best = max(cand, key=lambda a: dims[a] / blk[a])
        blk[best] *= 2
    out = (blk["t"], blk["h"], blk["w"])
    if out[0] * out[1] * out[2] != tile:
        raise ValueError(f"no {tile}-token block divides ({t},{h},{w})")
    return out


def space_time_reorder_index(t: int, h: int, w: int, block: Optional[tuple] = None,
                             native_axis_order: tuple = AXES, device=None) -> torch.Tensor:
    """perm (new position -> native token) grouping each (bt, bh, bw)
    neighbourhood of the (t, h, w) latent grid into one 128-token block."""
    if block is None:
        block = choose_local_block(t, h, w)
    bt, bh, bw = block
    if bt * bh * bw != QUERY_TILE:
        raise ValueError(f"block {block} product != {QUERY_TILE}")
    if t % bt or h % bh or w % bw:
        raise ValueError(f"block {block} does not divide grid ({t},{h},{w})")
    if sorted(native_axis_order) != sorted(AXES):
        raise ValueError(f"native_axis_order must be a permutation of {AXES}")
    dims = {"t": t, "h": h, "w": w}
    native = torch.arange(t * h * w, device=device).reshape(*[dims[a] for a in native_axis_order])
    grid = native.permute(*[native_axis_order.index(a) for a in AXES])          # (t, h, w)
    blocks = grid.reshape(t // bt, bt, h // bh, bh, w // bw, bw).permute(0, 2, 4, 1, 3, 5)
    return blocks.reshape(-1).contiguous()


def apply_token_permutation(x: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """x[:, perm] for a (B, S, H, D) tensor."""
    return x.index_select(1, perm)


def invert_permutation(perm: torch.Tensor) -> torch.Tensor:
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel(), device=perm.device, dtype=perm.dtype)
    return inv


def block_diagonal_mass(q, k, perm, *, sm_scale: Optional[float] = None, n_heads: int = 4,
                        n_query_tiles: int = 8) -> float:
    """Mean softmax mass a sampled 128-row tile puts on its own 128-key block
    after permuting Q/K by ``perm`` (a locality score for reorder layouts)."""
    _, s, h, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    nb = s // KEY_BLOCK
    hs = min(n_heads, h)
    qh = q[0].index_select(0, perm).permute(1, 0, 2)[:hs].float().contiguous()
    kh = k[0].index_select(0, perm).permute(1, 0, 2)[:hs].float().contiguous()
    picks = sorted(set(torch.linspace(0, nb - 1, steps=min(n_query_tiles, nb)).round().long().tolist()))
    vals = []
    for i in picks:
        sc = torch.matmul(qh[:, i * QUERY_TILE:(i + 1) * QUERY_TILE], kh.transpose(1, 2).contiguous()) * sm_scale
        mass = torch.softmax(sc, dim=-1).view(hs, QUERY_TILE, nb, KEY_BLOCK).sum(-1)
        vals.append(float(mass[..., i].mean()))
    return float(sum(vals) / max(1, len(vals)))


# ---- quantisation rules ----------------------------------------------------------------


@dataclass
class QuantStats:
    saturation_rate: float = 0.0
    underflow_zero_rate: float = 0.0
    roundtrip_rmse: float = 0.0


def _check_gpu(x: torch.Tensor, what: str) -> None:
    if not x.is_cuda:
        raise ValueError(f"{what} requires CUDA tensors")


def _head_quant(x3: torch.Tensor, mm_dtype: Optional[torch.dtype], want_deq: bool):
    """(deq fp32 or None, deq rounded to mm_dtype as fp32 or None, scale (H,), QuantStats)."""
    s, h, d = x3.shape
    x3 = x3.contiguous()
    if x3.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"unsupported dtype {x3.dtype}")
    dev = x3.device
    deq = torch.empty(s, h, d, dtype=torch.float32, device=dev) if want_deq else None
    deq_mm = torch.empty(s, h, d, dtype=torch.float32, device=dev) if mm_dtype is not None else None
    scale = torch.empty(h, dtype=torch.float32, device=dev)
    ws = torch.empty(h, dtype=torch.int32, device=dev)
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    sqerr = torch.zeros(1, dtype=torch.float64, device=dev)
    lib = _lib.load()
    _lib.check(lib.lbfq_head_fp8_quant(x3.data_ptr(), _lib.DTYPE_CODE[x3.dtype], s, h, d, _lib.ptr(deq),
                                       _lib.ptr(deq_mm), int(mm_dtype == torch.bfloat16), scale.data_ptr(),
                                       ws.data_ptr(), counts.data_ptr(), sqerr.data_ptr(),
                                       _lib.stream_handle(dev)), "head_fp8_quant")
    n = x3.numel()
    c = counts.tolist()
    stats = QuantStats(c[0] / n, c[1] / n, math.sqrt(float(sqerr.item()) / n))
    return deq, deq_mm, scale, stats


def fake_quant_per_head(x: torch.Tensor):
    """Per-head static-amax E4M3 fake quant of an (S, H, D) tensor:
    (dequantised fp32, scale (1, H, 1), QuantStats)."""
    if x.ndim != 3:
        raise ValueError(f"expected (S, H, D); got {tuple(x.shape)}")
    _check_gpu(x, "fake_quant_per_head")
    deq, _, scale, stats = _head_quant(x, None, True)
    return deq, scale.view(1, -1, 1), stats


def static_p_quant(p: torch.Tensor) -> torch.Tensor:
    """The static softmax-weight rule dequant(quant(p * 256, e4m3)) / 256."""
    return (p * P_STATIC_SCALE).to(torch.float8_e4m3fn).to(torch.float32) / P_STATIC_SCALE


def static_p_quant_with_stats(p: torch.Tensor):
    """(p_q, saturated count, underflow-to-zero count, squared error sum, count)."""
    scaled = p * P_STATIC_SCALE
    q = scaled.to(torch.float8_e4m3fn).to(torch.float32)
    deq = q / P_STATIC_SCALE
    return (deq, int((scaled.abs() > E4M3_MAX).sum()), int(((q == 0) & (scaled != 0)).sum()),
            float((deq - p).pow(2).sum()), p.numel())


# ---- skip predicate ---------------------------------------------------------------------


@dataclass
class SkipDiagnostics:
    skip_threshold: float
    skip_rate: float = 0.0
    force_keep_count: int = 0
    dropped_mass_mean: float = 0.0
    dropped_mass_median: float = 0.0
    dropped_mass_p95: float = 0.0
    dropped_mass_max: float = 0.0


@dataclass
class SimulationResult:
    outputs: dict = field(default_factory=dict)
    skip_outputs: dict = field(default_factory=dict)
    quant_stats: dict = field(default_factory=dict)
    skip_diagnostics: dict = field(default_factory=dict)
    peak_memory_bytes: int = 0


def _log_threshold(skip_threshold: float) -> float:
    return -math.inf if skip_threshold <= 0.0 else math.log(skip_threshold)


def running_row_max(block_max: torch.Tensor) -> torch.Tensor:
    """Cumulative max over the block axis (the online running row max)."""
    return torch.cummax(block_max, dim=-1).values


def blasst_keep_mask(block_max: torch.Tensor, log_threshold: float) -> torch.Tensor:
    """Per-row keep: block_max_j - running_max_j >= log(threshold)."""
    return (block_max - running_row_max(block_max)) >= log_threshold


def blasst_tile_keep_mask(block_max_per_row: torch.Tensor, log_threshold: float) -> torch.Tensor:
    """Tile keep from (..., rows, n_blocks) per-row block maxima: a block is kept
    iff some row keeps it (max over rows of the per-row margin)."""
    margin = block_max_per_row - running_row_max(block_max_per_row)
    return margin.amax(dim=-2) >= log_threshold


# ---- the simulator ----------------------------------------------------------------------


class _Sim:
    """Launch helpers over (S, H, D) fp32 operands of one workload."""

    def __init__(self, s: int, h: int, d: int, sm_scale: float, device):
        self.s, self.h, self.d, self.sm, self.dev = s, h, d, sm_scale, device
        self.nb = s // KEY_BLOCK
        self.lib = _lib.load()
        self.stream = _lib.stream_handle(device)

    def scan(self, q, k):
        fm = torch.empty(self.h, self.s, dtype=torch.float32, device=self.dev)
        n = self.h * self.nb * self.nb
        tm = torch.empty(n, dtype=torch.int32, device=self.dev)
        tb = torch.empty(n, dtype=torch.int32, device=self.dev)
        _lib.check(self.lib.lbfq_blasst_scan(q.data_ptr(), k.data_ptr(), self.s, self.h, self.d, self.sm,
                                             fm.data_ptr(), tm.data_ptr(), tb.data_ptr(), self.stream),
                   "blasst_scan")
        return fm, tm, tb

    def keep(self, tm, tb, thresholds):
        logt = torch.tensor([_log_threshold(t) for t in thresholds], dtype=torch.float32, device=self.dev)
        keep = torch.empty(len(thresholds), self.h, self.nb, self.nb, dtype=torch.uint8, device=self.dev)
        counts = torch.zeros(2 * len(thresholds), dtype=torch.int64, device=self.dev)
        _lib.check(self.lib.lbfq_blasst_keep(tm.data_ptr(), tb.data_ptr(), self.h, self.s, logt.data_ptr(),
                                             len(thresholds), keep.data_ptr(), counts.data_ptr(), self.stream),
                   "blasst_keep")
        return keep, counts.tolist()

    def attend(self, q, k, v, fm, mode, round_p, keep=None, dropped=False, p_stats=False):
        out = torch.empty(self.s, self.h, self.d, dtype=torch.float32, device=self.dev)
        drop = torch.empty(self.h, self.s, dtype=torch.float32, device=self.dev) if dropped else None
        pc = torch.zeros(2, dtype=torch.int64, device=self.dev) if p_stats else None
        pe = torch.zeros(1, dtype=torch.float64, device=self.dev) if p_stats else None
        p = _lib.BlasstAttendParams()
        p.S, p.H, p.D = self.s, self.h, self.d
        p.q, p.k, p.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
        p.sm_scale = self.sm
        p.mode, p.round_p_bf16 = mode, int(round_p)
        p.final_max = fm.data_ptr()
        p.keep = _lib.ptr(keep)
        p.out = out.data_ptr()
        p.dropped = _lib.ptr(drop)
        p.p_counts, p.p_sqerr = _lib.ptr(pc), _lib.ptr(pe)
        _lib.check(self.lib.lbfq_blasst_attend(p, self.stream), "blasst_attend")
        return out, drop, pc, pe


def _quantiles(dm: torch.Tensor):
    sd = dm.float().flatten().sort().values
    n = sd.numel()
    return (float(sd.mean()), float(sd[(n - 1) // 2]), float(sd[min(n - 1, int(0.95 * (n - 1)))]),
            float(sd[-1]))


def simulate_workload(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, skip_thresholds, levels=LADDER,
                      matmul_dtype: torch.dtype = torch.bfloat16,
                      collect_dropped_mass: bool = True) -> SimulationResult:
    """Run the ablation ladder over one (1, S, H, D) workload on the GPU.

    Operands enter the matmuls rounded to ``matmul_dtype`` (bf16 or fp32) with
    fp32 accumulation, as in the reference; D must be 64 or 128.
    """
    if q.ndim != 4 or q.shape[0] != 1:
        raise ValueError(f"expected (1, S, H, D); got {tuple(q.shape)}")
    if not q.is_cuda:
        raise ValueError("simulate_workload requires CUDA tensors")
    _, s, h, d = q.shape
    if s % QUERY_TILE != 0:
        raise ValueError(f"seqlen {s} must be a multiple of {QUERY_TILE}")
    if matmul_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"matmul_dtype must be bfloat16 or float32; got {matmul_dtype}")
    if d not in (64, 128):
        raise ValueError(f"head dim {d} not supported (64 or 128)")
    levels = list(levels)
    thresholds = list(skip_thresholds)
    want_skip = LEVEL_FP8_SKIP in levels and len(thresholds) > 0
    want_fp8 = any(lv in levels for lv in (LEVEL_FP8_QKV, LEVEL_FP8_STATIC_P, LEVEL_FP8_SKIP))
    round_p = matmul_dtype == torch.bfloat16
    dev = q.device
    sim = _Sim(s, h, d, 1.0 / math.sqrt(d), dev)
    torch.cuda.reset_peak_memory_stats(dev)
    result = SimulationResult()

    if LEVEL_REFERENCE in levels:
        qr, kr, vr = (t[0].to(matmul_dtype).float().contiguous() for t in (q, k, v))
        fm, _, _ = sim.scan(qr, kr)
        out, *_ = sim.attend(qr, kr, vr, fm, 0, round_p)
        result.outputs[LEVEL_REFERENCE] = out.view(1, s, h, d)
        del qr, kr, vr, fm

    if want_fp8:
        qd, kd, vd = [], [], []
        for name, t, dst in (("q", q, qd), ("k", k, kd), ("v", v, vd)):
            _, mm, _, st = _head_quant(t[0], matmul_dtype, False)
            dst.append(mm)
            result.quant_stats[name] = st
        qd, kd, vd = qd[0], kd[0], vd[0]
        fm, tm, tb = sim.scan(qd, kd)
        if LEVEL_FP8_QKV in levels:
            out, *_ = sim.attend(qd, kd, vd, fm, 1, round_p)
            result.outputs[LEVEL_FP8_QKV] = out.view(1, s, h, d)
        p_stats_done = False
        if LEVEL_FP8_STATIC_P in levels:
            out, _, pc, pe = sim.attend(qd, kd, vd, fm, 2, round_p, p_stats=True)
            result.outputs[LEVEL_FP8_STATIC_P] = out.view(1, s, h, d)
            p_stats_done = True
        if want_skip:
            keep, counts = sim.keep(tm, tb, thresholds)
            total_pairs = (s // QUERY_TILE) * h * sim.nb
            for i, th in enumerate(thresholds):
                stats_here = not p_stats_done and i == 0
                out, drop, pc_i, pe_i = sim.attend(qd, kd, vd, fm, 2, round_p, keep=keep[i],
                                                   dropped=collect_dropped_mass, p_stats=stats_here)
                if stats_here:
                    pc, pe = pc_i, pe_i
                    p_stats_done = True
                result.skip_outputs[th] = out.view(1, s, h, d)
                diag = SkipDiagnostics(skip_threshold=th, skip_rate=counts[2 * i] / max(1, total_pairs),
                                       force_keep_count=int(counts[2 * i + 1]))
                if collect_dropped_mass:
                    (diag.dropped_mass_mean, diag.dropped_mass_median, diag.dropped_mass_p95,
                     diag.dropped_mass_max) = _quantiles(drop)
                result.skip_diagnostics[th] = diag
        if p_stats_done:
            uf, cnt = pc.tolist()
            result.quant_stats["p"] = QuantStats(0.0, uf / max(1, cnt), math.sqrt(float(pe.item()) / max(1, cnt)))
    torch.cuda.synchronize(dev)
    result.peak_memory_bytes = int(torch.cuda.max_memory_allocated(dev))
    return result


__all__ = [
    "E4M3_MAX", "P_STATIC_SCALE", "QUERY_TILE", "KEY_BLOCK", "DENOM_FLOOR", "LEVEL_REFERENCE", "LEVEL_FP8_QKV",
    "LEVEL_FP8_STATIC_P", "LEVEL_FP8_SKIP", "LADDER", "MATH_BACKEND_SEQLEN_LIMIT", "FullMatrixAllocationError",
    "guard_no_full_matrix", "select_sdpa_backends", "sdpa_ground_truth", "choose_local_block",
    "space_time_reorder_index", "block_diagonal_mass", "apply_token_permutation", "invert_permutation",
    "QuantStats", "fake_quant_per_head", "static_p_quant", "static_p_quant_with_stats", "SkipDiagnostics",
    "SimulationResult", "running_row_max", "blasst_keep_mask", "blasst_tile_keep_mask", "simulate_workload",
]
