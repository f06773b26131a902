"""CPU restatement of the Q/K Hadamard rotation (test infrastructure only).

Follows ``hadamard.py:25-117`` of the reference (its torch fallback, which is
the path taken when ``fast-hadamard-transform`` is absent):

* signs: ``torch.Generator("cpu").manual_seed(seed)``,
  ``randint(0, 2, (H, D), int8) * 2 - 1`` (``hadamard.py:58-62``);
* ``x * sign`` in the input dtype (exact, the signs are +-1);
* FWHT in fp32, stages stride = 1, 2, 4, ...: ``(l, r) -> (l + r, l - r)``
  (``hadamard.py:36-44``);
* ``* fp32(1/sqrt(next_pow2(D)))`` then cast back to the input dtype (RNE).

Pinned by ``tests/test_oracle_hadamard.py``: H H^T = I on one-hot inputs,
agreement with ``scipy.linalg.hadamard`` (Sylvester order), logits of
rotated Q/K equal the unrotated ones, and the committed sign fixture
``tests/golden/hadamard_signs_h40_d128_seed0.npy``.
"""

from __future__ import annotations

import math

import torch


def signs(h: int, d: int, seed: int) -> torch.Tensor:
    gen = torch.Generator(device="cpu").manual_seed(int(seed))
    s = torch.randint(0, 2, (h, d), generator=gen, dtype=torch.int8)
    return s.mul_(2).sub_(1)


def _next_pow2(x: int) -> int:
    return 1 << (x - 1).bit_length()


def fwht_last_dim(x: torch.Tensor, scale: float) -> torch.Tensor:
    d = x.shape[-1]
    y = x.reshape(-1, d).float().clone()
    stride = 1
    while stride < d:
        y = y.reshape(-1, d // (2 * stride), 2 * stride)
        left = y[..., :stride].clone()
        right = y[..., stride:2 * stride].clone()
        y[..., :stride] = left + right
        y[..., stride:2 * stride] = left - right
        y = y.reshape(-1, d)
        stride *= 2
    return (y * float(scale)).to(x.dtype).reshape(x.shape)


def apply_qk_hadamard(q: torch.Tensor, k: torch.Tensor, *, random_sign: bool = True, seed: int = 0):
    _, _, h, d = q.shape
    qw, kw = q.contiguous(), k.contiguous()
    if random_sign:
        sg = signs(h, d, seed).view(1, 1, h, d)
        qw = qw * sg.to(q.dtype)
        kw = kw * sg.to(k.dtype)
    scale = 1.0 / math.sqrt(float(_next_pow2(d)))
    return fwht_last_dim(qw, scale), fwht_last_dim(kw, scale)
