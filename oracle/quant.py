"""CPU restatement of the reference quantisers (test infrastructure only).

Follows ``quant_triton.py`` of the reference:

* ``fp8_block_quant``       -- ``quant_triton.py:26-77``
* ``fp8_per_channel_quant`` -- ``quant_triton.py:134-176``
* ``mxfp8_qk_quant``        -- ``quant_triton.py:221-271``
* ``mxfp8_v_quant``         -- ``quant_triton.py:322-369``
* the four dequantisers     -- ``quant_triton.py:80-131, 179-218, 274-319, 372-416``

Arithmetic: input -> fp32; ``amax = max(max|x|, fp32(1e-4))``;
``sc = amax / 448`` (IEEE fp32 division); codes = E4M3(clamp(x / sc, +-448)).
MX scales are ``2^clamp(ceil(log2(amax/448)), -127, 127)``; the exponent is
computed exactly from the fp32 bits of ``amax/448`` (for bf16/fp16 inputs this
equals the reference's ``tl.ceil(tl.log2(.))``: ``amax/448`` is either an exact
power of two or at least 1/224 away from one in relative terms).

Pinned by ``tests/test_oracle_quant.py``: codes round-trip through
``torch.float8_e4m3fn``; the amax element maps to +-448; an all-zero block
gives scale 1e-4/448 and codes 0; MX scales are exact powers of two with the
block max in [224, 448]; dequant(quant(x)) error bounds.  All arrays are
``torch`` CPU tensors; codes are returned as ``torch.uint8``.
"""

from __future__ import annotations

import numpy as np
import torch

from . import fp8

FP8_MAX = np.float32(448.0)
AMAX_FLOOR = np.float32(1e-4)


def _encode_t(x: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(fp8.encode(x.contiguous().numpy()))


def _decode_t(c: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(fp8.decode(c.contiguous().numpy()))


def ceil_log2_exact(r: np.ndarray) -> np.ndarray:
    """ceil(log2(r)) for positive finite normal fp32 ``r``, exact from bits."""
    r = np.ascontiguousarray(np.asarray(r, dtype=np.float32))
    u = r.view(np.uint32)
    e = (u >> 23).astype(np.int64) - 127
    mant = u & 0x7FFFFF
    return e + (mant != 0).astype(np.int64)


def _mx_scale(amax: torch.Tensor) -> torch.Tensor:
    r = (amax / torch.tensor(FP8_MAX)).numpy()
    e = np.clip(ceil_log2_exact(r), -127, 127)
    return torch.from_numpy(np.ldexp(np.float32(1.0), e).astype(np.float32))


def _quant_with_scale(x: torch.Tensor, sc: torch.Tensor) -> torch.Tensor:
    xq = torch.clamp(x / sc, -448.0, 448.0)
    return _encode_t(xq)


def fp8_block_quant(t: torch.Tensor, block_s: int = 128):
    """(B,S,H,D) -> codes uint8 (B,S,H,D), scale fp32 (B,S/block_s,H)."""
    b, s, h, d = t.shape
    if s % block_s:
        raise ValueError(f"S={s} must be divisible by block_s={block_s}")
    x = t.float().reshape(b, s // block_s, block_s, h, d)
    amax = x.abs().amax(dim=(2, 4)).clamp_min(float(AMAX_FLOOR))  # (b, n, h)
    sc = amax / torch.tensor(FP8_MAX)
    codes = _quant_with_scale(x, sc[:, :, None, :, None])
    return codes.reshape(b, s, h, d), sc


def fp8_block_dequant(codes: torch.Tensor, scale: torch.Tensor, block_s: int = 128,
                      dtype=torch.float32) -> torch.Tensor:
    b, s, h, d = codes.shape
    v = _decode_t(codes).reshape(b, s // block_s, block_s, h, d)
    return (v * scale[:, :, None, :, None]).reshape(b, s, h, d).to(dtype)


def fp8_per_channel_quant(t: torch.Tensor, block_s: int = 128):
    """(B,S,H,D) -> codes, scale fp32 (B,H,D)."""
    x = t.float()
    amax = x.abs().amax(dim=1).clamp_min(float(AMAX_FLOOR))  # (b, h, d)
    sc = amax / torch.tensor(FP8_MAX)
    return _quant_with_scale(x, sc[:, None]), sc


def fp8_per_channel_dequant(codes, scale, block_s: int = 128, dtype=torch.float32):
    return (_decode_t(codes) * scale[:, None]).to(dtype)


def mxfp8_qk_quant(t: torch.Tensor, block_d: int = 32):
    """(B,S,H,D) -> codes, pow2 scale fp32 (B,S,H,D/block_d)."""
    b, s, h, d = t.shape
    if d % block_d:
        raise ValueError(f"D={d} must be divisible by block_d={block_d}")
    x = t.float().reshape(b, s, h, d // block_d, block_d)
    amax = x.abs().amax(dim=4).clamp_min(float(AMAX_FLOOR))
    sc = _mx_scale(amax)
    codes = _quant_with_scale(x, sc[..., None])
    return codes.reshape(b, s, h, d), sc


def mxfp8_qk_dequant(codes, scale, block_d: int = 32, dtype=torch.float32):
    b, s, h, d = codes.shape
    v = _decode_t(codes).reshape(b, s, h, d // block_d, block_d)
    return (v * scale[..., None]).reshape(b, s, h, d).to(dtype)


def mxfp8_v_quant(t: torch.Tensor, block_s: int = 32):
    """(B,S,H,D) -> codes, pow2 scale fp32 (B,S/block_s,H,D)."""
    b, s, h, d = t.shape
    if s % block_s:
        raise ValueError(f"S={s} must be divisible by block_s={block_s}")
    x = t.float().reshape(b, s // block_s, block_s, h, d)
    amax = x.abs().amax(dim=2).clamp_min(float(AMAX_FLOOR))
    sc = _mx_scale(amax)
    codes = _quant_with_scale(x, sc[:, :, None])
    return codes.reshape(b, s, h, d), sc


def mxfp8_v_dequant(codes, scale, block_s: int = 32, dtype=torch.float32):
    b, s, h, d = codes.shape
    v = _decode_t(codes).reshape(b, s // block_s, block_s, h, d)
    return (v * scale[:, :, None]).reshape(b, s, h, d).to(dtype)


def decode(codes: torch.Tensor) -> torch.Tensor:
    return _decode_t(codes)
