"""Thin typed wrappers around the C ABI (one call = one or a few HIP launches).

Everything launches on the current torch stream of the tensors' device and
allocates its outputs with torch (the library itself never allocates).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib

AMAX_FLOOR_BITS = 0x38D1B717  # bits of fp32(1e-4), the reference's amax floor


def _dt(t: torch.Tensor) -> int:
    try:
        return _lib.DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16") from None


@dataclass
class RowSource:
    """A (B,S,H,D) NHD tensor as seen through an optional row gather and an
    optional mean subtraction (the lazily-applied preprocess of one operand)."""

    x: torch.Tensor
    gather: torch.Tensor | None = None     # (B*H, S) int32: source row of each output row
    sub_mode: int = _lib.SUB_NONE
    sub: torch.Tensor | None = None        # fp32 (B,H,D) or (B,S/G,H,D)
    sub_block: int = 0

    @property
    def shape(self):
        return self.x.shape


def rowtile(src: RowSource, *, R: int, smoothed: torch.Tensor | None = None, smoothed_stage: int = 0,
            signs: torch.Tensor | None = None, hadamard: bool = False, had_scale: float = 1.0,
            quant_mode: int = _lib.Q_NONE, codes: torch.Tensor | None = None, codes_layout: int = _lib.LAYOUT_NHD,
            codes_spitch: int = 0, scale: torch.Tensor | None = None, scale_strides=(0, 0, 0, 0),
            amax_table: torch.Tensor | None = None, mx_block: int = 32, scale_e8m0: bool = False) -> None:
    lib = _lib.load()
    x = src.x
    b, s, h, d = x.shape
    p = _lib.RowTileParams()
    p.x = x.data_ptr(); p.x_dtype = _dt(x)
    p.B, p.S, p.H, p.D = b, s, h, d
    p.R = int(R)
    p.gather = _lib.ptr(src.gather)
    p.sub_mode = src.sub_mode; p.sub = _lib.ptr(src.sub); p.sub_block = int(src.sub_block)
    p.smoothed = _lib.ptr(smoothed)
    p.hadamard = 1 if hadamard else 0; p.signs = _lib.ptr(signs); p.had_scale = float(had_scale)
    p.quant_mode = quant_mode
    p.codes = _lib.ptr(codes); p.codes_layout = codes_layout; p.codes_spitch = int(codes_spitch)
    p.scale = _lib.ptr(scale)
    p.sc_b, p.sc_s, p.sc_h, p.sc_d = (int(v) for v in scale_strides)
    p.amax_table = _lib.ptr(amax_table)
    p.mx_block = int(mx_block)
    p.smoothed_stage = int(smoothed_stage)
    p.scale_e8m0 = 1 if scale_e8m0 else 0
    _lib.check(lib.lbfq_rowtile(p, _lib.stream_handle(x.device)), "lbfq_rowtile")


def colsum_mean(x: torch.Tensor, chunk: int, gather: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 means of consecutive `chunk`-row groups: (B, S/chunk, H, D)."""
    lib = _lib.load()
    b, s, h, d = x.shape
    out = torch.empty((b, (s + chunk - 1) // chunk, h, d), dtype=torch.float32, device=x.device)
    _lib.check(lib.lbfq_colsum(x.data_ptr(), _dt(x), b, s, h, d, int(chunk), _lib.ptr(gather), 1, None,
                               out.data_ptr(), _lib.stream_handle(x.device)), "lbfq_colsum")
    return out


def column_mean(x: torch.Tensor, chunk: int = 256) -> torch.Tensor:
    """fp32 mean over S per (b, h, d), fixed chunked fp64 order: (B, H, D)."""
    lib = _lib.load()
    b, s, h, d = x.shape
    nchunk = (s + chunk - 1) // chunk
    part = torch.empty((b, nchunk, h, d), dtype=torch.float64, device=x.device)
    mean = torch.empty((b, h, d), dtype=torch.float32, device=x.device)
    st = _lib.stream_handle(x.device)
    _lib.check(lib.lbfq_colsum(x.data_ptr(), _dt(x), b, s, h, d, int(chunk), None, 0, part.data_ptr(), None, st),
               "lbfq_colsum")
    _lib.check(lib.lbfq_colsum_finalize(part.data_ptr(), b, nchunk, h, d, s, mean.data_ptr(), st),
               "lbfq_colsum_finalize")
    return mean


def channel_amax(src: RowSource, tile: int = 1024) -> torch.Tensor:
    """Per-(b,h,d) max |x| over S (floored at fp32(1e-4)) as uint32 fp32 bits.

    One workgroup per `tile` rows of a head (the row-tile kernel's largest
    tile: fewest workgroups and atomics; 64.5 against 72 us at tile 256 for
    40 x 32768 x 128 bf16 on an MI355X).  The max does not depend on the
    tiling, so every tile size gives the same bits.
    """
    lib = _lib.load()
    b, s, h, d = src.x.shape
    table = torch.empty((b, h, d), dtype=torch.int32, device=src.x.device)
    _lib.check(lib.lbfq_fill_u32(table.data_ptr(), table.numel(), AMAX_FLOOR_BITS,
                                 _lib.stream_handle(src.x.device)), "lbfq_fill_u32")
    rowtile(src, R=tile, quant_mode=_lib.Q_CHANNEL_AMAX, amax_table=table)
    return table


def dequant(codes_u8: torch.Tensor, scale: torch.Tensor, mode: int, block: int, dtype: torch.dtype) -> torch.Tensor:
    lib = _lib.load()
    b, s, h, d = codes_u8.shape
    out = torch.empty((b, s, h, d), dtype=dtype, device=codes_u8.device)
    _lib.check(lib.lbfq_dequant(codes_u8.data_ptr(), scale.data_ptr(), b, s, h, d, mode, int(block),
                                out.data_ptr(), _dt(out), _lib.stream_handle(codes_u8.device)), "lbfq_dequant")
    return out


def kmeans(x: torch.Tensor, k: int, iters: int, seed: int):
    """-> (labels, order, inverse) int32 (B*H, S)."""
    lib = _lib.load()
    b, s, h, d = x.shape
    ws = torch.empty(int(lib.lbfq_kmeans_workspace_bytes(b, s, h, d, int(k))), dtype=torch.uint8, device=x.device)
    labels = torch.empty((b * h, s), dtype=torch.int32, device=x.device)
    order = torch.empty_like(labels)
    inverse = torch.empty_like(labels)
    _lib.check(lib.lbfq_kmeans(x.data_ptr(), _dt(x), b, s, h, d, int(k), int(iters), int(seed) & (2**64 - 1),
                               ws.data_ptr(), labels.data_ptr(), order.data_ptr(), inverse.data_ptr(),
                               _lib.stream_handle(x.device)), "lbfq_kmeans")
    return labels, order, inverse


def qmk(qm: torch.Tensor, k: RowSource, sm_scale: float, *, s_pitch: int, want_bias: bool = True,
        want_rowmax: bool = True, k_quant: tuple | None = None):
    """bias (B,H,G,s_pitch) = qm.K_s * sm_scale and rowmax (B,H,G) = max_n bias,
    with K_s the smoothed (and gathered) K described by ``k``: no K_s tensor is
    materialised when ``k`` subtracts a per-(b,h) column mean.

    k_quant = (codes (B,H,P,D) uint8, scale (B,H,S/block) fp32, block): also
    quantise K_s in fp8_block mode in the same pass (bf16 K only; the codes and
    scales equal the row-tile quantiser's bit for bit)."""
    lib = _lib.load()
    x = k.x
    b, s, h, d = x.shape
    g = qm.shape[1]
    dev = x.device
    if k.sub_mode not in (_lib.SUB_NONE, _lib.SUB_COLVEC):
        raise ValueError("qmk: K smoothing is a per-(b,h) column mean")
    bias = None
    if want_bias:
        alloc = torch.zeros if s_pitch > s else torch.empty
        bias = alloc((b, h, g, s_pitch), dtype=torch.float32, device=dev)
    rowmax = torch.empty((b, h, g), dtype=torch.float32, device=dev) if want_rowmax else None
    qm = qm.contiguous().float()
    mean = k.sub if k.sub_mode == _lib.SUB_COLVEC else None
    split = torch.empty((b, h, 3, g, d // 2), dtype=torch.int32, device=dev) if x.dtype == torch.bfloat16 else None
    if k_quant is None:
        _lib.check(lib.lbfq_qmk(qm.data_ptr(), x.data_ptr(), _dt(x), _lib.ptr(k.gather), _lib.ptr(mean), b, s, h, d,
                                g, float(sm_scale), _lib.ptr(bias), int(s_pitch), _lib.ptr(rowmax), _lib.ptr(split),
                                _lib.stream_handle(dev)), "lbfq_qmk")
    else:
        codes, kscale, blk = k_quant
        if codes.dtype != torch.uint8 or codes.shape[:2] != (b, h) or codes.shape[3] != d or not codes.is_contiguous():
            raise ValueError("qmk: K codes must be a contiguous (B,H,P,D) uint8 tensor")
        if kscale.dtype != torch.float32 or kscale.shape != (b, h, s // blk) or not kscale.is_contiguous():
            raise ValueError("qmk: K scales must be a contiguous (B,H,S/block) fp32 tensor")
        _lib.check(lib.lbfq_qmk_kquant(qm.data_ptr(), x.data_ptr(), _dt(x), _lib.ptr(k.gather), _lib.ptr(mean), b, s,
                                       h, d, g, float(sm_scale), _lib.ptr(bias), int(s_pitch), _lib.ptr(rowmax),
                                       _lib.ptr(split), codes.data_ptr(), codes.shape[2], kscale.data_ptr(), int(blk),
                                       _lib.stream_handle(dev)), "lbfq_qmk_kquant")
    return bias, rowmax


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def hadamard_scale(d: int) -> float:
    return 1.0 / math.sqrt(float(1 << (d - 1).bit_length()))
