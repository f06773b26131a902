"""CPU restatement of the k-means token reorder (test infrastructure only).

Reorder plumbing follows ``kmeans.py:44-135`` of the reference:
``x = t.permute(0,2,1,3).reshape(B*H,S,D).float()``; labels from the
clustering; ``order = argsort(labels, stable=True)``;
``inverse[order[j]] = j``; ``t_reordered[j] = t[order[j]]``;
``apply_kv_permutation`` gathers K rows by V's order.

The clustering itself is this build's deterministic Lloyd specification
(``kmeans_ref.c``); flash-kmeans label parity is unpinned (absent
dependency).  ``kmeans_labels_py`` is an independent slow Python restatement
used to pin the C code.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libkmeans_ref.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build as _build
            _build.build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.lbfq_ref_kmeans.restype = ctypes.c_int
        lib.lbfq_ref_kmeans.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p,
        ]
        lib.lbfq_ref_kmeans_mix.restype = ctypes.c_uint64
        lib.lbfq_ref_kmeans_mix.argtypes = [ctypes.c_uint64] * 4
        _lib = lib
    return _lib


def kmeans_labels(x_bsd: np.ndarray, k: int, iters: int, seed: int):
    """x: (BH, S, D) fp32 -> (labels int32 (BH,S), centroids fp32 (BH,k,D))."""
    x = np.ascontiguousarray(x_bsd, dtype=np.float32)
    bh, s, d = x.shape
    labels = np.empty((bh, s), dtype=np.int32)
    cent = np.empty((bh, k, d), dtype=np.float32)
    rc = _load().lbfq_ref_kmeans(x.ctypes.data, bh, s, d, k, iters, seed & (2**64 - 1),
                                 labels.ctypes.data, cent.ctypes.data)
    if rc != 0:
        raise ValueError(f"kmeans oracle rejected k={k} for S={s}")
    return labels, cent


def mix(seed: int, bh: int, k: int, j: int) -> int:
    m = 2**64 - 1
    z = (seed + 0x9E3779B97F4A7C15 * (bh * k + j + 1)) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def kmeans_labels_py(x_sd: np.ndarray, k: int, iters: int, seed: int, bh: int = 0):
    """Slow scalar restatement of the same specification for one slice."""
    x = np.asarray(x_sd, dtype=np.float32)
    s, d = x.shape
    stride = s // k
    c = np.stack([x[j * stride + mix(seed, bh, k, j) % stride] for j in range(k)]).astype(np.float32)

    def fma(a, b, acc):  # exact fused multiply-add on fp32 via fp64 + exact check
        import fractions
        r = fractions.Fraction(float(a)) * fractions.Fraction(float(b)) + fractions.Fraction(float(acc))
        return np.float32(_round_fraction_to_f32(r))

    def assign(c):
        cn = []
        for j in range(k):
            a = np.float32(0)
            for dd in range(d):
                a = fma(c[j, dd], c[j, dd], a)
            cn.append(a)
        lab = np.zeros(s, dtype=np.int32)
        for t in range(s):
            best, bj = np.float32(np.inf), 0
            for j in range(k):
                a = np.float32(0)
                for dd in range(d):
                    a = fma(x[t, dd], c[j, dd], a)
                sc = fma(np.float32(-2.0), a, cn[j])
                if sc < best:
                    best, bj = sc, j
            lab[t] = bj
        return lab

    lab = assign(c) if iters <= 0 else None
    for _ in range(iters):
        lab = assign(c)
        tot = np.zeros((k, d), dtype=np.float64)
        cnt = np.zeros(k, dtype=np.int64)
        for c0 in range(0, s, 1024):
            part = np.zeros((k, d), dtype=np.float64)
            for t in range(c0, min(c0 + 1024, s)):
                part[lab[t]] += x[t].astype(np.float64)
                cnt[lab[t]] += 1
            tot += part
        for j in range(k):
            if cnt[j]:
                c[j] = (tot[j] / cnt[j]).astype(np.float32)
    return lab, c


def _round_fraction_to_f32(r) -> float:
    """Round an exact rational to the nearest fp32 (ties to even)."""
    import fractions
    if r == 0:
        return 0.0
    f64 = float(r)  # nearest double
    # resolve double-rounding: pick the fp32 neighbour(s) of f64 and compare exactly
    f = np.float32(f64)
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    best = min(cands, key=lambda c: (abs(fractions.Fraction(float(c)) - r),
                                     int(np.array(c, dtype=np.float32).view(np.uint32)) & 1))
    return float(best)


def reorder_from_labels(labels: torch.Tensor):
    """labels (BH,S) int -> (order int64, inverse int64) per kmeans.py:84-87."""
    order = torch.argsort(labels.to(torch.int64), dim=1, stable=True)
    pos = torch.arange(labels.shape[1]).expand_as(order)
    inverse = torch.empty_like(order)
    inverse.scatter_(1, order, pos)
    return order, inverse


def kmeans_reorder_tokens(t: torch.Tensor, *, n_clusters: int, max_iters: int = 10, seed: int = 0):
    """(B,S,H,D) -> dict(tensor_reordered, order, inverse_order, labels)."""
    b, s, h, d = t.shape
    if n_clusters <= 0 or n_clusters > s:
        raise ValueError(f"n_clusters must be in [1, S]; got {n_clusters} for S={s}")
    x = t.permute(0, 2, 1, 3).reshape(b * h, s, d).contiguous().float()
    lab, _ = kmeans_labels(x.numpy(), n_clusters, max_iters, seed)
    labels = torch.from_numpy(lab).to(torch.int64)
    order, inverse = reorder_from_labels(labels)
    xr = torch.gather(x, 1, order.unsqueeze(-1).expand(-1, -1, d))
    tr = xr.reshape(b, h, s, d).permute(0, 2, 1, 3).to(t.dtype).contiguous()
    return dict(tensor_reordered=tr, order=order, inverse_order=inverse, labels=labels)


def apply_kv_permutation(t: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    b, s, h, d = t.shape
    tb = t.permute(0, 2, 1, 3).reshape(b * h, s, d).contiguous()
    tr = torch.gather(tb, 1, order.unsqueeze(-1).expand(-1, -1, d))
    return tr.reshape(b, h, s, d).permute(0, 2, 1, 3).contiguous().to(t.dtype)
