"""Q/K/V smoothing on gfx950.

Same signatures, outputs and error messages as the reference's
``preprocess.py`` (smooth_k :38-57, smooth_v_per_block :135-166,
group_mean_q :169-193).  Means are accumulated in fp64 in a fixed
sequential order (per 256-row chunk, then over chunks, for the K mean) and
rounded once to fp32; the smoothed tensor is ``fp32(x) - mean`` rounded to
the input dtype.
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import _lib
from ._ops import RowSource, colsum_mean, column_mean, rowtile


def smooth_k(k: torch.Tensor, block_s: int = 256) -> Tuple[torch.Tensor, torch.Tensor]:
    """K-mean subtraction over the S axis.

    Returns ``(k_smoothed, k_mean)``; ``k_mean`` is FP32 ``(B, H, D)`` and
    ``k_smoothed`` has the dtype of ``k``.  ``block_s`` is accepted for API
    compatibility; the reduction order is fixed (256-row chunks).
    """
    if k.ndim != 4 or not k.is_cuda:
        raise ValueError(f"k must be 4-D NHD on CUDA; got {tuple(k.shape)} on {k.device}")
    b, s, h, d = k.shape
    if d not in (64, 128):
        raise ValueError(f"D must be 64 or 128; got {d}")
    k = k.contiguous()
    mean = column_mean(k)
    out = torch.empty_like(k)
    rowtile(RowSource(k, sub_mode=_lib.SUB_COLVEC, sub=mean), R=64, smoothed=out)
    return out, mean


def group_mean_q(q: torch.Tensor, block_q: int = 256) -> Tuple[torch.Tensor, torch.Tensor]:
    """Q centering by groups along S.

    Returns ``(q_centered, qm)`` where ``qm`` is FP32 with shape
    ``(B, S / block_q, H, D)``.
    """
    if q.ndim != 4 or not q.is_cuda:
        raise ValueError(f"q must be 4-D NHD on CUDA; got {tuple(q.shape)} on {q.device}")
    b, s, h, d = q.shape
    if s % block_q != 0:
        raise ValueError(f"S={s} must be divisible by block_q={block_q}")
    if d not in (64, 128):
        raise ValueError(f"D must be 64 or 128; got {d}")
    q = q.contiguous()
    qm = colsum_mean(q, block_q)
    out = torch.empty_like(q)
    rowtile(RowSource(q, sub_mode=_lib.SUB_BLOCKVEC, sub=qm, sub_block=block_q), R=64, smoothed=out)
    return out, qm


def smooth_v_per_block(v: torch.Tensor, block_s: int = 64) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-S-block V mean smoothing.

    Returns ``(v_centered, v_alpha)`` where ``v_alpha`` is FP32 with shape
    ``(B, S/block_s, H, D)``; the attention folds the block means back in.
    """
    if v.ndim != 4 or not v.is_cuda:
        raise ValueError(f"v must be 4-D NHD on CUDA; got {tuple(v.shape)} on {v.device}")
    b, s, h, d = v.shape
    if s % block_s != 0:
        raise ValueError(f"S={s} must be divisible by block_s={block_s}")
    if d not in (64, 128):
        raise ValueError(f"D must be 64 or 128; got {d}")
    v = v.contiguous()
    alpha = colsum_mean(v, block_s)
    out = torch.empty_like(v)
    rowtile(RowSource(v, sub_mode=_lib.SUB_BLOCKVEC, sub=alpha, sub_block=block_s), R=64, smoothed=out)
    return out, alpha


__all__ = ["smooth_k", "group_mean_q", "smooth_v_per_block"]
