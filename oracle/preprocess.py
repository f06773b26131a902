"""CPU restatement of the smoothing kernels (test infrastructure only).

Follows ``preprocess.py`` of the reference:

* ``smooth_k``           -- ``preprocess.py:10-57``  (K -= mean over S)
* ``group_mean_q``       -- ``preprocess.py:60-91, 169-193`` (Q -= mean per group)
* ``smooth_v_per_block`` -- ``preprocess.py:94-166`` (V -= mean per S-block)

The reference accumulates in fp32 in Triton's (unspecified) reduction order.
This build fixes one order so GPU and CPU agree bit for bit on every input:

* sums are accumulated in fp64, strictly sequentially in row order, starting
  from +0.0;
* ``smooth_k`` sums each 256-row chunk sequentially, then adds the chunk
  partials sequentially in chunk order (a final partial chunk for ragged S);
* the mean is ``fp32(sum / n)`` (fp64 division, one rounding to fp32);
* the smoothed value is ``fp32(x) - mean`` in fp32, rounded (RNE) to the
  output dtype (the input dtype, as in the reference).

Pinned by ``tests/test_oracle_preprocess.py``: means equal exact rational
means (``fractions.Fraction``) rounded to fp32 on small inputs; the
chunk-order rule is checked against a scalar loop; K smoothing leaves
softmax(QK^T) invariant; per-block means of the centred V are ~0.
"""

from __future__ import annotations

import numpy as np
import torch

SMOOTH_K_CHUNK = 256


def _seq_sum_rows(x64: np.ndarray, axis: int) -> np.ndarray:
    """Sequential fp64 sum along ``axis`` in index order, starting at +0.0."""
    x64 = np.moveaxis(x64, axis, 0)
    acc = np.zeros(x64.shape[1:], dtype=np.float64)
    for r in range(x64.shape[0]):
        acc = acc + x64[r]
    return acc


def k_mean(k: torch.Tensor) -> torch.Tensor:
    """(B,S,H,D) -> fp32 (B,H,D) per the fixed chunk order."""
    b, s, h, d = k.shape
    x = k.float().numpy().astype(np.float64)
    total = np.zeros((b, h, d), dtype=np.float64)
    for c0 in range(0, s, SMOOTH_K_CHUNK):
        part = _seq_sum_rows(x[:, c0:c0 + SMOOTH_K_CHUNK], axis=1)
        total = total + part
    return torch.from_numpy((total / float(s)).astype(np.float32))


def smooth_k(k: torch.Tensor):
    """Returns (k_smoothed in k.dtype, k_mean fp32 (B,H,D))."""
    mean = k_mean(k)
    out = (k.float() - mean[:, None]).to(k.dtype)
    return out, mean


def _block_mean(x: torch.Tensor, block: int) -> torch.Tensor:
    b, s, h, d = x.shape
    xb = x.float().numpy().astype(np.float64).reshape(b, s // block, block, h, d)
    sums = _seq_sum_rows(xb, axis=2)                  # (b, n, h, d)
    return torch.from_numpy((sums / float(block)).astype(np.float32))


def group_mean_q(q: torch.Tensor, block_q: int = 256):
    """Returns (q_centered in q.dtype, qm fp32 (B,S/block_q,H,D))."""
    b, s, h, d = q.shape
    if s % block_q:
        raise ValueError(f"S={s} must be divisible by block_q={block_q}")
    qm = _block_mean(q, block_q)
    out = (q.float() - qm.repeat_interleave(block_q, dim=1)).to(q.dtype)
    return out, qm


def smooth_v_per_block(v: torch.Tensor, block_s: int = 64):
    """Returns (v_centered in v.dtype, v_alpha fp32 (B,S/block_s,H,D))."""
    b, s, h, d = v.shape
    if s % block_s:
        raise ValueError(f"S={s} must be divisible by block_s={block_s}")
    alpha = _block_mean(v, block_s)
    out = (v.float() - alpha.repeat_interleave(block_s, dim=1)).to(v.dtype)
    return out, alpha
