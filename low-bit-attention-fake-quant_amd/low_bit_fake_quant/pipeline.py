"""Legacy ``prepare_qkv`` pipeline (reference ``pipeline.py:19-110``).

Order as in the reference: Q k-means -> smoothing (with the qm.K_s
correction tensor in ``cfg.correction_dtype``) -> optional Hadamard ->
quantise Q/K/V.  Every step runs on this package's HIP kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ._ops import RowSource, qmk
from .config import QuantConfig
from .hadamard import apply_qk_hadamard
from .kmeans import KMeansReorderResult, q_kmeans_reorder
from .preprocess import group_mean_q, smooth_k
from .quant import fp8_block_quant, fp8_per_channel_quant, mxfp8_qk_quant, mxfp8_v_quant


@dataclass
class PreparedQKV:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    q_scale: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    qm: torch.Tensor | None = None
    k_mean: torch.Tensor | None = None
    correction: torch.Tensor | None = None
    kmeans: KMeansReorderResult | None = None


def _validate_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q/k/v shapes must match; got {q.shape}, {k.shape}, {v.shape}")
    if q.ndim != 4:
        raise ValueError(f"q/k/v must be 4-D NHD; got {q.shape}")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q/k/v must live on CUDA")


def prepare_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cfg: QuantConfig) -> PreparedQKV:
    """Run the configured QKV preprocessing and quantization pipeline."""
    _validate_qkv(q, k, v)
    q_work, k_work, v_work = q.contiguous(), k.contiguous(), v.contiguous()
    kmeans = None
    if cfg.q_kmeans_k is not None:
        kmeans = q_kmeans_reorder(q_work, n_clusters=cfg.q_kmeans_k, max_iters=cfg.q_kmeans_iters,
                                  seed=cfg.q_kmeans_seed)
        q_work = kmeans.q_reordered
    qm = k_mean = correction = None
    if cfg.smoothing == "k_only":
        k_work, k_mean = smooth_k(k_work)
    elif cfg.smoothing == "full":
        k_work, k_mean = smooth_k(k_work)
        q_work, qm = group_mean_q(q_work, block_q=cfg.q_smooth_block_size)
        bias, _ = qmk(qm, RowSource(k_work), 1.0, s_pitch=k_work.shape[1], want_rowmax=False)   # (B,H,G,S)
        correction = bias.permute(0, 2, 1, 3).contiguous().to(cfg.correction_dtype)  # (B,G,H,S)
    elif cfg.smoothing != "off":
        raise ValueError(f"unsupported smoothing mode: {cfg.smoothing!r}")
    if cfg.qk_hadamard:
        q_work, k_work = apply_qk_hadamard(q_work, k_work, random_sign=cfg.qk_hadamard_random_sign,
                                           seed=cfg.qk_hadamard_seed)
    if cfg.qk_quant == "fp8_block":
        q_quant, q_scale = fp8_block_quant(q_work, block_s=cfg.fp8_block_size)
        k_quant, k_scale = fp8_block_quant(k_work, block_s=cfg.fp8_block_size)
    elif cfg.qk_quant == "mxfp8":
        q_quant, q_scale = mxfp8_qk_quant(q_work, block_d=cfg.mxfp8_block_size)
        k_quant, k_scale = mxfp8_qk_quant(k_work, block_d=cfg.mxfp8_block_size)
    else:
        raise ValueError(f"unsupported qk_quant: {cfg.qk_quant!r}")
    if cfg.v_quant == "fp8_channel":
        v_quant, v_scale = fp8_per_channel_quant(v_work)
    elif cfg.v_quant == "fp8_block":
        v_quant, v_scale = fp8_block_quant(v_work, block_s=cfg.v_fp8_block_size)
    elif cfg.v_quant == "mxfp8":
        v_quant, v_scale = mxfp8_v_quant(v_work, block_s=cfg.v_mxfp8_block_size)
    else:
        raise ValueError(f"unsupported v_quant: {cfg.v_quant!r}")
    return PreparedQKV(q=q_quant, k=k_quant, v=v_quant, q_scale=q_scale, k_scale=k_scale, v_scale=v_scale, qm=qm,
                       k_mean=k_mean, correction=correction, kmeans=kmeans)
