"""Token k-means reorder on gfx950.

Same API as the reference's ``kmeans.py`` (KMeansReorderResult :26-41,
kmeans_reorder_tokens :44-95, q_kmeans_reorder :98-110, v_kmeans_reorder
:113-124, apply_kv_permutation :127-135).  The clustering runs on this
library's own deterministic Lloyd kernels (the reference calls the external
flash-kmeans package); the order is the stable argsort of the labels and
``inverse_order`` its inverse, as in the reference.  ``order``,
``inverse_order`` and ``labels`` are int64 ``(B*H, S)`` like the reference;
int32 copies used by the kernels are kept alongside.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from ._ops import RowSource, kmeans as _kmeans, rowtile


@dataclass
class KMeansReorderResult:
    tensor_reordered: torch.Tensor
    order: torch.Tensor
    inverse_order: torch.Tensor
    labels: torch.Tensor
    order_i32: torch.Tensor | None = field(default=None, repr=False)
    inverse_i32: torch.Tensor | None = field(default=None, repr=False)

    @property
    def q_reordered(self) -> torch.Tensor:  # pragma: no cover - trivial
        return self.tensor_reordered

    @property
    def v_reordered(self) -> torch.Tensor:  # pragma: no cover - trivial
        return self.tensor_reordered


def gather_rows(t: torch.Tensor, order_i32: torch.Tensor) -> torch.Tensor:
    """out[b, s, h] = t[b, order[b*H+h, s], h] for an NHD tensor."""
    t = t.contiguous()
    out = torch.empty_like(t)
    rowtile(RowSource(t, gather=order_i32), R=64, smoothed=out)
    return out


def kmeans_labels(t: torch.Tensor, *, n_clusters: int, max_iters: int = 10, seed: int = 0):
    """int32 (labels, order, inverse), each (B*H, S), without materialising the reorder."""
    if t.ndim != 4 or not t.is_cuda:
        raise ValueError(f"t must be 4-D NHD on CUDA; got {tuple(t.shape)} on {t.device}")
    b, s, h, d = t.shape
    if n_clusters <= 0 or n_clusters > s:
        raise ValueError(f"n_clusters must be in [1, S]; got {n_clusters} for S={s}")
    return _kmeans(t.contiguous(), n_clusters, max_iters, seed)


def make_result(t: torch.Tensor, labels: torch.Tensor, order: torch.Tensor, inverse: torch.Tensor,
                reordered: torch.Tensor | None = None) -> KMeansReorderResult:
    if reordered is None:
        reordered = gather_rows(t, order)
    return KMeansReorderResult(tensor_reordered=reordered, order=order.to(torch.int64),
                               inverse_order=inverse.to(torch.int64), labels=labels.to(torch.int64),
                               order_i32=order, inverse_i32=inverse)


def kmeans_reorder_tokens(
    t: torch.Tensor,
    *,
    n_clusters: int,
    max_iters: int = 10,
    seed: int = 0,
    chunk_tokens: int = 4096,  # kept for backward compatibility; unused
) -> KMeansReorderResult:
    """Cluster tokens of ``t`` (B, S, H, D) per (B, H) and return a reorder result."""
    del chunk_tokens
    labels, order, inverse = kmeans_labels(t, n_clusters=n_clusters, max_iters=max_iters, seed=seed)
    return make_result(t, labels, order, inverse)


def q_kmeans_reorder(q: torch.Tensor, *, n_clusters: int = 32, max_iters: int = 10, seed: int = 0,
                     chunk_tokens: int = 4096) -> KMeansReorderResult:
    """Cluster Q tokens per (B, H) and reorder them; attention output rows must be
    inverse-permuted to restore the original Q order."""
    return kmeans_reorder_tokens(q, n_clusters=n_clusters, max_iters=max_iters, seed=seed,
                                 chunk_tokens=chunk_tokens)


def v_kmeans_reorder(v: torch.Tensor, *, n_clusters: int = 32, max_iters: int = 10,
                     seed: int = 0) -> KMeansReorderResult:
    """Cluster V tokens per (B, H) and reorder; callers must co-permute K with ``order``."""
    return kmeans_reorder_tokens(v, n_clusters=n_clusters, max_iters=max_iters, seed=seed)


def apply_kv_permutation(t: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    """Apply a (B*H, S) permutation along S of a (B, S, H, D) tensor."""
    if t.ndim != 4:
        raise ValueError(f"t must be (B,S,H,D); got {tuple(t.shape)}")
    return gather_rows(t, order.to(device=t.device, dtype=torch.int32).contiguous())


__all__ = [
    "KMeansReorderResult", "apply_kv_permutation", "kmeans_reorder_tokens", "q_kmeans_reorder",
    "v_kmeans_reorder",
]
