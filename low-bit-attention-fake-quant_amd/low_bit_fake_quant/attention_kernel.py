"""Host side of the FP8-MFMA P-requant attention kernel.

Mirrors the guards and BLASST fill parsing of the reference's
``fake_quant_attention_triton`` (``attention_triton.py:463-624, 674-714``),
with the same messages, and launches ``lbfq_attention_fwd``.  Unlike the
reference wrapper it takes FP8 codes + scales (the kernel multiplies codes on
the matrix cores) rather than pre-dequantised bf16 tensors.
"""

from __future__ import annotations

import math
import re

import torch

from . import _lib

_BLASST_FILL_ZERO = 0
_BLASST_FILL_MAX = 1
_BLASST_FILL_MEAN = 2
_BLASST_FILL_LOGN = 3
_BLASST_FILL_SAMPLE8 = 4
_BLASST_FILL_THR = 5
_BLASST_FILL_UTA = 6

KERNEL_BLOCK_N = 64   # keys per tile of the gfx950 kernel
KERNEL_BLOCK_NS = (64, 128)  # block_n values: one or two tiles per row-max / BLASST decision


def parse_blasst_fill(mode: str | None, *, alpha: float, uta_bins: int) -> tuple[int, float, int]:
    """Map BLASST fill strings to (kind, alpha, uta_bins) (attention_triton.py:674-714)."""
    if mode is None or mode == "zero":
        return _BLASST_FILL_ZERO, float(alpha), 1
    if mode == "max":
        return _BLASST_FILL_MAX, float(alpha), 1
    if mode.startswith("max_a"):
        return _BLASST_FILL_MAX, float(mode[len("max_a"):]), 1
    if mode == "mean":
        return _BLASST_FILL_MEAN, float(alpha), 1
    if mode.startswith("mean_a"):
        return _BLASST_FILL_MEAN, float(mode[len("mean_a"):]), 1
    if mode == "logn":
        return _BLASST_FILL_LOGN, float(alpha), 1
    if mode == "sample8":
        return _BLASST_FILL_SAMPLE8, float(alpha), 1
    if mode.startswith("sample8_a"):
        return _BLASST_FILL_SAMPLE8, float(mode[len("sample8_a"):]), 1
    if mode == "thr":
        return _BLASST_FILL_THR, float(alpha), 1
    if mode.startswith("thr_a"):
        return _BLASST_FILL_THR, float(mode[len("thr_a"):]), 1
    if mode == "uta":
        if uta_bins <= 0:
            raise ValueError(f"blasst_uta_bins must be > 0; got {uta_bins}")
        return _BLASST_FILL_UTA, float(alpha), int(uta_bins)
    uta = re.fullmatch(r"uta(\d+)(?:_a([0-9]+(?:\.[0-9]+)?))?", mode)
    if uta:
        bins = int(uta.group(1))
        if bins <= 0:
            raise ValueError(f"UTA bin count must be > 0; got {bins}")
        parsed_alpha = float(uta.group(2)) if uta.group(2) is not None else float(alpha)
        return _BLASST_FILL_UTA, parsed_alpha, bins
    raise ValueError(f"unknown blasst_fill_mode: {mode!r}")


def resolve_p_mode(cfg) -> str:
    p_mode = cfg.p_quant
    if p_mode == "auto":
        p_mode = "mx" if cfg.v_quant == "mxfp8" else "elementwise"
    return p_mode


def validate_kernel_config(cfg, *, s: int, d: int, has_qm: bool, has_v_alpha: bool) -> None:
    """Reference guards (attention_triton.py:478-611) plus this kernel's limits."""
    block_m, block_n = cfg.p_requant_block_m, cfg.p_requant_block_n
    if has_v_alpha:
        vsb = cfg.v_smooth_block_size
        if vsb <= 0:
            raise ValueError("v_smooth_block must be > 0 when v_alpha is given")
        if vsb < block_n or vsb % block_n != 0:
            raise ValueError(f"v_smooth_block ({vsb}) must be >= block_n ({block_n}) "
                             "and an integer multiple of block_n")
        if s % vsb != 0:
            raise ValueError(f"S ({s}) must be divisible by v_smooth_block ({vsb})")
    if has_qm:
        qsb = cfg.q_smooth_block_size
        if qsb <= 0:
            raise ValueError("q_smooth_block must be > 0 with qm_bhgd")
        if qsb < block_m or qsb % block_m != 0:
            raise ValueError(f"q_smooth_block ({qsb}) must be >= block_m ({block_m}) "
                             "and an integer multiple of block_m")
        if s % qsb != 0:
            raise ValueError(f"S ({s}) must be divisible by q_smooth_block ({qsb})")
    if cfg.v_quant == "fp8_block":
        vb = cfg.v_fp8_block_size
        if vb <= 0:
            raise ValueError("v_block_size must be > 0 when v_block_scale_bsh is given")
        if vb < block_n or vb % block_n != 0:
            raise ValueError(f"v_block_size ({vb}) must be >= block_n ({block_n}) and an integer multiple of block_n")
        if s % vb != 0:
            raise ValueError(f"S ({s}) must be divisible by v_block_size ({vb})")
    p_mode = resolve_p_mode(cfg)
    if p_mode == "mx":
        p_mx = cfg.p_mx_block_n if cfg.p_mx_block_n > 0 else cfg.v_mxfp8_block_size
        if p_mx <= 0:
            raise ValueError("p_mx_block_n must be > 0 when p_quant_mode='mx'")
        if p_mx != block_n:
            raise ValueError(f"p_mx_block_n ({p_mx}) currently must equal block_n ({block_n}); "
                             "sub-block scaling within a K block is not implemented")
    elif p_mode not in ("elementwise", "dynamic"):
        raise ValueError(f"unknown p_quant_mode: {p_mode!r}")
    if cfg.blasst_lambda is not None:
        if not (0.0 < float(cfg.blasst_lambda) < 1.0):
            raise ValueError(f"blasst_lambda must be in (0, 1); got {cfg.blasst_lambda}")
        kind, _, bins = parse_blasst_fill(cfg.blasst_fill, alpha=cfg.blasst_fill_alpha, uta_bins=cfg.blasst_uta_bins)
        if kind == _BLASST_FILL_UTA and block_n % bins != 0:
            raise ValueError(f"blasst UTA bins ({bins}) must divide block_n ({block_n})")
    elif cfg.blasst_fill not in ("zero", None):
        raise ValueError("blasst_fill_mode requires blasst_lambda")
    # ---- limits of the gfx950 kernel -------------------------------------
    def pow2(x):
        return x > 0 and (x & (x - 1)) == 0

    if block_n not in KERNEL_BLOCK_NS:
        raise ValueError(f"the gfx950 P-requant kernel runs p_requant_block_n in {KERNEL_BLOCK_NS}; got {block_n}")
    if block_m <= 0:
        raise ValueError(f"p_requant_block_m must be > 0; got {block_m}")
    if cfg.qk_quant == "mxfp8" and cfg.mxfp8_block_size != 32:
        raise ValueError("the gfx950 MX attention consumes E8M0 scales per 32 elements along D; "
                         f"mxfp8_block_size must be 32, got {cfg.mxfp8_block_size}")
    if cfg.qk_quant == "fp8_block" and not (pow2(cfg.fp8_block_size) and cfg.fp8_block_size >= 16):
        raise ValueError(f"fp8_block_size must be a power of two >= 16 for the gfx950 kernel; got {cfg.fp8_block_size}")
    if cfg.v_quant == "mxfp8" and not (pow2(cfg.v_mxfp8_block_size) and cfg.v_mxfp8_block_size >= KERNEL_BLOCK_N):
        raise ValueError(f"v_mxfp8_block_size must be a power of two >= {KERNEL_BLOCK_N} for the gfx950 kernel; "
                         f"got {cfg.v_mxfp8_block_size}")
    if cfg.v_quant == "fp8_block" and not pow2(cfg.v_fp8_block_size):
        raise ValueError(f"v_fp8_block_size must be a power of two for the gfx950 kernel; got {cfg.v_fp8_block_size}")
    if cfg.v_quant == "fp8_block" and cfg.v_fp8_block_size > 512:
        raise ValueError("v_fp8_block_size above 512 is not supported by the gfx950 V quantiser")
    if has_v_alpha and not pow2(cfg.v_smooth_block_size):
        raise ValueError(f"v_smooth_block_size must be a power of two for the gfx950 kernel; "
                         f"got {cfg.v_smooth_block_size}")
    if has_qm and not (pow2(cfg.q_smooth_block_size) and cfg.q_smooth_block_size >= 32):
        raise ValueError(f"q_smooth_block_size must be a power of two >= 32 for the gfx950 kernel; "
                         f"got {cfg.q_smooth_block_size}")


def _attn_params(ops, cfg, sm_scale: float) -> "_lib.AttnParams":
    """lbfq_attn_params for the quantised operands (no output, stats or skip buffers)."""
    p = _lib.AttnParams()
    p.B, p.H, p.S, p.D = ops.b, ops.h, ops.s, ops.d
    p.s_pitch = ops.P
    p.q_codes, p.k_codes, p.v_codes_t = ops.q_codes.data_ptr(), ops.k_codes.data_ptr(), ops.v_codes_t.data_ptr()
    p.qk_mx = 1 if cfg.qk_quant == "mxfp8" else 0
    p.q_scale, p.k_scale = ops.q_scale.data_ptr(), ops.k_scale.data_ptr()
    p.qk_block = cfg.fp8_block_size if cfg.qk_quant == "fp8_block" else 0
    p.v_kind = ops.v_kind
    p.v_scale = ops.v_scale.data_ptr()
    p.v_block = ops.v_block
    p_mode = resolve_p_mode(cfg)
    p.p_mode = {"elementwise": 0, "mx": 1, "dynamic": 2}[p_mode]
    p.sm_scale = float(sm_scale)
    p.p_max_offset = int(cfg.p_max_offset)
    p.block_m = int(cfg.p_requant_block_m)
    p.qk_bias = _lib.ptr(ops.bias)
    p.q_group = int(cfg.q_smooth_block_size) if ops.bias is not None or ops.rowmax is not None else 0
    p.rowmax_est = _lib.ptr(ops.rowmax)
    p.rowmax_dynamic = 1 if p_mode == "dynamic" else 0
    p.v_alpha = _lib.ptr(ops.v_alpha)
    p.v_smooth_block = int(cfg.v_smooth_block_size) if ops.v_alpha is not None else 0
    if cfg.blasst_lambda is not None:
        kind, alpha, bins = parse_blasst_fill(cfg.blasst_fill, alpha=cfg.blasst_fill_alpha,
                                              uta_bins=cfg.blasst_uta_bins)
        p.blasst_lambda = float(cfg.blasst_lambda)
        p.blasst_fill, p.blasst_fill_alpha, p.blasst_uta_bins = kind, float(alpha), int(bins)
    else:
        p.blasst_lambda = 0.0
        p.blasst_fill, p.blasst_fill_alpha, p.blasst_uta_bins = 0, 1.0, 1
    p.out_row_map = _lib.ptr(ops.out_row_map)
    p.v_tile_colsum = _lib.ptr(getattr(ops, "v_colsum", None))
    p.block_n = int(cfg.p_requant_block_n)
    return p


def v_tile_colsum(v_codes_t: torch.Tensor, v_scale: torch.Tensor, v_kind: int, v_block: int, s: int) -> torch.Tensor:
    """Column sums of the V^T codes (B,H,D,P) over each 64-key tile (MX V:
    scaled by its E8M0 block scales): (B*H, P/64, D) fp32."""
    lib = _lib.load()
    b, h, d, P = v_codes_t.shape
    out = torch.empty((b * h, P // 64, d), dtype=torch.float32, device=v_codes_t.device)
    _lib.check(lib.lbfq_v_tile_colsum(v_codes_t.data_ptr(), b * h, s, P, d, int(v_kind), v_scale.data_ptr(),
                                      int(v_block), out.data_ptr(), _lib.stream_handle(v_codes_t.device)),
               "lbfq_v_tile_colsum")
    return out


def launch_attention(ops, cfg, sm_scale: float, out_dtype: torch.dtype, *, return_blasst_stats: bool = False,
                     return_row_skips: bool = False, return_wave_tiles: bool = False,
                     rowmax_init: torch.Tensor | None = None):
    """Run the attention kernel on quantised operands; returns NHD output, then
    (when asked) the BLASST stats (ceil(S/block_m), B*H, 2), the per-row
    skipped K-block counts (B*H, S) in output-row order, and per wave of 32
    reordered query rows the number of block_n-key decision blocks (64-key
    tiles at block_n = 64, 128-key blocks at 128) that every row of the wave
    skipped (softmax and PV elided) and that some row skipped,
    (B*H, ceil(S/128)*4, 2) int32.  ``rowmax_init`` (B*H, S) fp32: the
    initial row max of each (reordered) query row in log2 units
    (attention_triton.py rowmax_init_bhs * log2 e); not with a qm_k estimate."""
    lib = _lib.load()
    dev = ops.q_codes.device
    out = torch.empty((ops.b, ops.s, ops.h, ops.d), dtype=out_dtype, device=dev)
    p = _attn_params(ops, cfg, sm_scale)
    if rowmax_init is not None:
        if rowmax_init.shape != (ops.b * ops.h, ops.s) or rowmax_init.dtype != torch.float32 or \
                rowmax_init.device != dev or not rowmax_init.is_contiguous():
            raise ValueError(f"rowmax_init must be a contiguous (B*H, S) fp32 tensor on {dev}")
        if ops.rowmax is not None:
            raise ValueError("rowmax_init_bhs and rowmax_est_bhs are mutually exclusive")
        p.rowmax_init = rowmax_init.data_ptr()
    stats = row_skips = wave_tiles = None
    if cfg.blasst_lambda is not None:
        if return_blasst_stats:
            nblk = (ops.s + cfg.p_requant_block_m - 1) // cfg.p_requant_block_m
            stats = torch.zeros((nblk, ops.b * ops.h, 2), dtype=torch.float32, device=dev)
            p.blasst_stats = stats.data_ptr()
        if return_row_skips:
            row_skips = torch.zeros((ops.b * ops.h, ops.s), dtype=torch.float32, device=dev)
            p.blasst_row_skips = row_skips.data_ptr()
        if return_wave_tiles:
            nw = (ops.s + 127) // 128 * 4
            wave_tiles = torch.zeros((ops.b * ops.h, nw, 2), dtype=torch.int32, device=dev)
            p.blasst_wave_tiles = wave_tiles.data_ptr()
    p.out = out.data_ptr()
    p.out_dtype = _lib.DTYPE_CODE[out_dtype]
    _lib.check(lib.lbfq_attention_fwd(p, _lib.stream_handle(dev)), "lbfq_attention_fwd")
    res = [out]
    if return_blasst_stats:
        res.append(stats)
    if return_row_skips:
        res.append(row_skips)
    if return_wave_tiles:
        res.append(wave_tiles)
    return res[0] if len(res) == 1 else tuple(res)


def attention_scores(ops, cfg, sm_scale: float, rows: torch.Tensor | None = None) -> torch.Tensor:
    """The attention kernel's scores in log2 units for the given query rows of
    its (reordered) row order: (B*H, len(rows), S) fp32 (diagnostic)."""
    lib = _lib.load()
    dev = ops.q_codes.device
    if rows is None:
        rows = torch.arange(ops.s, device=dev, dtype=torch.int32)
    rows = rows.to(device=dev, dtype=torch.int32).contiguous()
    if rows.numel() == 0 or int(rows.min()) < 0 or int(rows.max()) >= ops.s:
        raise ValueError(f"rows must be non-empty indices in [0, {ops.s})")
    u = torch.empty((ops.b * ops.h, rows.numel(), ops.s), dtype=torch.float32, device=dev)
    p = _attn_params(ops, cfg, sm_scale)
    _lib.check(lib.lbfq_attention_scores(p, rows.data_ptr(), rows.numel(), u.data_ptr(), _lib.stream_handle(dev)),
               "lbfq_attention_scores")
    return u


def attention_flops(s: int, h: int, d: int, b: int = 1) -> float:
    """Algorithmic FLOPs of one non-causal attention: 4 * S^2 * D * H * B."""
    return 4.0 * float(s) * float(s) * float(d) * float(h) * float(b)


__all__ = ["parse_blasst_fill", "validate_kernel_config", "launch_attention", "attention_scores",
           "attention_flops", "resolve_p_mode", "math"]
