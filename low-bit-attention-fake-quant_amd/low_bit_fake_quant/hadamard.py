"""Orthonormal (random-sign) Hadamard rotation of Q/K along D on gfx950.

Same API as the reference's ``hadamard.py`` (fast_hadamard_available :16-19,
hadamard_transform_last_dim :50-55, apply_qk_hadamard :77-117).  The
transform is the in-register butterfly of the row-tile kernel with the
reference torch fallback's arithmetic (``hadamard.py:25-47``): signs applied
in the input dtype, stages stride 1, 2, ..., D/2 in fp32 as (l + r, l - r),
times fp32(1/sqrt(D)), rounded back to the input dtype.
"""

from __future__ import annotations

import math
from functools import lru_cache
from typing import Callable

import torch

from . import _lib
from ._ops import RowSource, hadamard_scale, rowtile

try:  # pragma: no cover - reported for API parity only; never used for compute
    import fast_hadamard_transform as _fht  # noqa: F401
    _FHT = True
except Exception:  # noqa: BLE001
    _FHT = False


def fast_hadamard_available() -> bool:
    """Whether Dao-AILab fast-hadamard-transform is importable (not used here)."""
    return _FHT


@lru_cache(maxsize=128)
def _cached_cpu_signs(h: int, d: int, seed: int) -> torch.Tensor:
    gen = torch.Generator(device="cpu").manual_seed(int(seed))
    signs = torch.randint(0, 2, (h, d), generator=gen, dtype=torch.int8)
    return signs.mul_(2).sub_(1)


_device_signs: dict = {}


def qk_signs_device(h: int, d: int, seed: int, device) -> torch.Tensor:
    """(H, D) int8 +-1 signs on ``device`` (host generator, cached)."""
    key = (h, d, int(seed), str(device))
    t = _device_signs.get(key)
    if t is None:
        t = _cached_cpu_signs(h, d, seed).to(device)
        _device_signs[key] = t
    return t


def hadamard_transform_last_dim(x: torch.Tensor, *, scale: float) -> torch.Tensor:
    """Unnormalised FWHT over the last dimension times ``scale`` (last dim 64 or 128)."""
    d = x.shape[-1]
    if d not in (64, 128):
        raise ValueError(f"hadamard_transform_last_dim supports a last dimension of 64 or 128; got {d}")
    if not x.is_cuda:
        raise ValueError("hadamard_transform_last_dim expects a CUDA tensor")
    xv = x.contiguous().reshape(1, -1, 1, d)
    out = torch.empty_like(xv)
    rowtile(RowSource(xv), R=64, hadamard=True, had_scale=float(scale), smoothed=out, smoothed_stage=1)
    return out.reshape(x.shape)


def apply_qk_hadamard(
    q: torch.Tensor,
    k: torch.Tensor,
    *,
    random_sign: bool = True,
    seed: int = 0,
    transform: Callable[[torch.Tensor], torch.Tensor] | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate Q/K by the same orthonormal Hadamard basis along head dim.

    ``x' = (x * sign) @ H / sqrt(D)`` per head with shared signs, so
    ``(Q R) @ (K R).T == Q @ K.T`` before quantisation.
    """
    if q.shape != k.shape:
        raise ValueError(f"q/k shapes must match; got {tuple(q.shape)} and {tuple(k.shape)}")
    if q.ndim != 4:
        raise ValueError(f"q/k must be NHD tensors; got {tuple(q.shape)}")
    if not (q.is_cuda and k.is_cuda):
        raise ValueError("q/k Hadamard rotation expects CUDA tensors")
    _, _, h, d = q.shape
    if d <= 0:
        raise ValueError("head dimension must be positive")
    if transform is not None:
        qw, kw = q.contiguous(), k.contiguous()
        if random_sign:
            sg = _cached_cpu_signs(h, d, seed).to(device=q.device, dtype=q.dtype).view(1, 1, h, d)
            qw = qw * sg
            kw = kw * sg.to(dtype=k.dtype)
        return transform(qw), transform(kw)
    if d not in (64, 128):
        raise ValueError(f"head dimension must be 64 or 128; got {d}")
    signs = qk_signs_device(h, d, seed, q.device) if random_sign else None
    scale = hadamard_scale(d)
    outs = []
    for t in (q, k):
        t = t.contiguous()
        o = torch.empty_like(t)
        rowtile(RowSource(t), R=64, hadamard=True, signs=signs, had_scale=scale, smoothed=o, smoothed_stage=1)
        outs.append(o)
    return outs[0], outs[1]


__all__ = ["apply_qk_hadamard", "fast_hadamard_available", "hadamard_transform_last_dim"]
