"""FP8 / MXFP8 quantisers and dequantisers on gfx950.

Same signatures, shapes, dtypes and error messages as the reference's
``quant_triton.py`` (fp8_block_quant :61-77, fp8_block_dequant :111-131,
fp8_per_channel_quant :163-176, fp8_per_channel_dequant :200-218,
mxfp8_qk_quant :255-271, mxfp8_qk_dequant :300-319, mxfp8_v_quant :354-369,
mxfp8_v_dequant :398-416).  Codes are ``torch.float8_e4m3fn``; scales fp32.
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import _lib
from ._ops import RowSource, channel_amax, dequant, rowtile


def _check_nhd(t: torch.Tensor, *, name: str = "tensor") -> tuple[int, int, int, int]:
    if t.ndim != 4:
        raise ValueError(f"{name} must be 4-D NHD (B, S, H, D); got {tuple(t.shape)}")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on CUDA; got {t.device}")
    b, s, h, d = t.shape
    if d not in (64, 128):
        raise ValueError(f"{name}.shape[-1] must be 64 or 128; got {d}")
    return b, s, h, d


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8)


def fp8_block_quant(t: torch.Tensor, block_s: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """FP32-scale FP8 e4m3fn quantization per (B, S/block_s, H)."""
    b, s, h, d = _check_nhd(t)
    if s % block_s != 0:
        raise ValueError(f"S={s} must be divisible by block_s={block_s}")
    t = t.contiguous()
    out = torch.empty_like(t, dtype=torch.float8_e4m3fn)
    scale = torch.empty((b, s // block_s, h), dtype=torch.float32, device=t.device)
    rowtile(RowSource(t), R=block_s, quant_mode=_lib.Q_FP8_BLOCK, codes=_u8(out), scale=scale,
            scale_strides=(scale.stride(0), scale.stride(1), scale.stride(2), 0))
    return out, scale


def fp8_block_dequant(fp8: torch.Tensor, scale: torch.Tensor, block_s: int = 128, *,
                      dtype: torch.dtype = torch.float32) -> torch.Tensor:
    b, s, h, d = _check_nhd(fp8, name="fp8")
    if fp8.dtype != torch.float8_e4m3fn:
        raise TypeError(f"fp8 must have dtype torch.float8_e4m3fn; got {fp8.dtype}")
    if tuple(scale.shape) != (b, s // block_s, h):
        raise ValueError(f"scale must have shape {(b, s // block_s, h)}; got {tuple(scale.shape)}")
    return dequant(_u8(fp8.contiguous()), scale.contiguous().float(), _lib.DQ_BLOCK, block_s, dtype)


def fp8_per_channel_quant(t: torch.Tensor, block_s: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """FP32-scale FP8 e4m3fn quantization for V, one scale per (B, H, D)."""
    b, s, h, d = _check_nhd(t)
    t = t.contiguous()
    out = torch.empty_like(t, dtype=torch.float8_e4m3fn)
    scale = torch.empty((b, h, d), dtype=torch.float32, device=t.device)
    src = RowSource(t)
    table = channel_amax(src)
    rowtile(src, R=64, quant_mode=_lib.Q_CHANNEL, codes=_u8(out), scale=scale,
            scale_strides=(scale.stride(0), 0, scale.stride(1), scale.stride(2)), amax_table=table)
    return out, scale


def fp8_per_channel_dequant(fp8: torch.Tensor, scale: torch.Tensor, block_s: int = 128, *,
                            dtype: torch.dtype = torch.float32) -> torch.Tensor:
    b, s, h, d = _check_nhd(fp8, name="fp8")
    if tuple(scale.shape) != (b, h, d):
        raise ValueError(f"scale must have shape {(b, h, d)}; got {tuple(scale.shape)}")
    return dequant(_u8(fp8.contiguous()), scale.contiguous().float(), _lib.DQ_CHANNEL, 0, dtype)


def mxfp8_qk_quant(t: torch.Tensor, block_d: int = 32) -> Tuple[torch.Tensor, torch.Tensor]:
    """MXFP8-style Q/K quantization along D, scale shape (B, S, H, D/block_d)."""
    b, s, h, d = _check_nhd(t)
    if d % block_d != 0:
        raise ValueError(f"D={d} must be divisible by block_d={block_d}")
    t = t.contiguous()
    out = torch.empty_like(t, dtype=torch.float8_e4m3fn)
    scale = torch.empty((b, s, h, d // block_d), dtype=torch.float32, device=t.device)
    rowtile(RowSource(t), R=64, quant_mode=_lib.Q_MX_QK, codes=_u8(out), scale=scale,
            scale_strides=scale.stride(), mx_block=block_d)
    return out, scale


def mxfp8_qk_dequant(fp8: torch.Tensor, scale: torch.Tensor, block_d: int = 32, *,
                     dtype: torch.dtype = torch.float32) -> torch.Tensor:
    b, s, h, d = _check_nhd(fp8, name="fp8")
    d_blocks = d // block_d
    if tuple(scale.shape) != (b, s, h, d_blocks):
        raise ValueError(f"scale must have shape {(b, s, h, d_blocks)}")
    return dequant(_u8(fp8.contiguous()), scale.contiguous().float(), _lib.DQ_MX_QK, block_d, dtype)


def mxfp8_v_quant(t: torch.Tensor, block_s: int = 32) -> Tuple[torch.Tensor, torch.Tensor]:
    """MXFP8-style V quantization along S, scale shape (B, S/block_s, H, D)."""
    b, s, h, d = _check_nhd(t)
    if s % block_s != 0:
        raise ValueError(f"S={s} must be divisible by block_s={block_s}")
    t = t.contiguous()
    out = torch.empty_like(t, dtype=torch.float8_e4m3fn)
    scale = torch.empty((b, s // block_s, h, d), dtype=torch.float32, device=t.device)
    rowtile(RowSource(t), R=block_s, quant_mode=_lib.Q_MX_V, codes=_u8(out), scale=scale,
            scale_strides=(scale.stride(0), scale.stride(1), scale.stride(2), scale.stride(3)))
    return out, scale


def mxfp8_v_dequant(fp8: torch.Tensor, scale: torch.Tensor, block_s: int = 32, *,
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
    b, s, h, d = _check_nhd(fp8, name="fp8")
    if tuple(scale.shape) != (b, s // block_s, h, d):
        raise ValueError(f"scale must have shape {(b, s // block_s, h, d)}")
    return dequant(_u8(fp8.contiguous()), scale.contiguous().float(), _lib.DQ_MX_V, block_s, dtype)


__all__ = [
    "fp8_block_quant", "fp8_block_dequant", "fp8_per_channel_quant", "fp8_per_channel_dequant",
    "mxfp8_qk_quant", "mxfp8_qk_dequant", "mxfp8_v_quant", "mxfp8_v_dequant",
]
