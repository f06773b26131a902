"""Small-shape FP8 P-requant probe (reference ``p_requant.py:44-73``).

``p_requant_rows(scores, sm_scale=..., p_max_offset=8)`` materialises, per row
of an unscaled ``(B, M, N)`` logit matrix,

* ``p = e4m3(2^((x - max_n x) * sm_scale * log2(e) + p_max_offset))``,
* ``row_sum = sum_n p`` (fp32, pre-quantisation values),
* ``lse = max * sm_scale + ln(row_sum) - p_max_offset * ln(2)``,

on one HIP kernel (one workgroup per row).  It writes all of P, so it is for
unit tests and probes, not for Wan-sized attention.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def _next_power_of_2(n: int) -> int:
    return 1 << (n - 1).bit_length() if n > 0 else 1


def p_requant_rows(
    scores: torch.Tensor,
    *,
    sm_scale: float,
    p_max_offset: int = 8,
    block_n: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns ``(p_fp8 (B,M,N) float8_e4m3fn, row_sum (B,M) fp32, lse (B,M) fp32)``."""
    if scores.ndim != 3 or not scores.is_cuda:
        raise ValueError(f"scores must be 3-D CUDA tensor; got {tuple(scores.shape)}")
    b, m, n = scores.shape
    if block_n is None:
        block_n = _next_power_of_2(n)
    if block_n < n:
        raise ValueError(f"block_n={block_n} must be >= N={n}")
    if scores.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"scores must be fp32/fp16/bf16; got {scores.dtype}")
    p = torch.empty_like(scores, dtype=torch.float8_e4m3fn)
    row_sum = torch.empty((b, m), dtype=torch.float32, device=scores.device)
    lse = torch.empty((b, m), dtype=torch.float32, device=scores.device)
    if scores.numel() == 0:
        return p, row_sum, lse
    lib = _lib.load()
    _lib.check(lib.lbfq_p_requant_rows(
        scores.data_ptr(), _lib.DTYPE_CODE[scores.dtype], b, m, n, *scores.stride(),
        p.data_ptr(), *p.stride(), row_sum.data_ptr(), lse.data_ptr(),
        float(sm_scale), int(p_max_offset), _lib.stream_handle(scores.device)), "p_requant_rows")
    return p, row_sum, lse


__all__ = ["p_requant_rows"]
