"""Pins the smoothing oracle (reference preprocess.py:10-193): means equal exact
rational means rounded to fp32, K smoothing leaves softmax invariant, centred V
blocks have zero mean."""

import fractions
import math
import os

import numpy as np
import pytest
import scipy.linalg
import torch

from conftest import REPO, cpu_randn
from oracle import fp8
from oracle import hadamard as ohad
from oracle import kmeans as okm
from oracle import preprocess as opre

GOLDEN = os.path.join(REPO, "tests", "golden")


# ---- smoothing means (reference preprocess.py:10-193) ------------------------


def _exact_mean_f32(col: np.ndarray) -> np.float32:
    tot = sum((fractions.Fraction(float(v)) for v in col), fractions.Fraction(0))
    r = tot / len(col)
    return np.float32(okm._round_fraction_to_f32(r))


def test_k_mean_equals_exact_rational_mean():
    k = cpu_randn(1, 600, 2, 64, seed=3) * 7  # 600: ragged last 256-row chunk
    m = opre.k_mean(k.bfloat16()).numpy()
    x = k.bfloat16().float().numpy()
    for h in range(2):
        for d in (0, 17, 63):
            assert m[0, h, d] == _exact_mean_f32(x[0, :, h, d])


def test_group_and_block_means_equal_exact_rational_means():
    q = cpu_randn(1, 512, 2, 64, seed=4)
    _, qm = opre.group_mean_q(q, block_q=256)
    _, va = opre.smooth_v_per_block(q, block_s=64)
    x = q.float().numpy()
    for g in range(2):
        assert qm[0, g, 1, 9].item() == _exact_mean_f32(x[0, g * 256:(g + 1) * 256, 1, 9])
    for blk in (0, 7):
        assert va[0, blk, 0, 33].item() == _exact_mean_f32(x[0, blk * 64:(blk + 1) * 64, 0, 33])


def test_k_smoothing_leaves_softmax_invariant():
    q = cpu_randn(1, 128, 2, 64, seed=5, dtype=torch.float32)
    k = cpu_randn(1, 128, 2, 64, seed=6, dtype=torch.float32) + 3.0
    ks, _ = opre.smooth_k(k)
    a = torch.softmax(torch.einsum("bshd,bthd->bhst", q, k), -1)
    b = torch.softmax(torch.einsum("bshd,bthd->bhst", q, ks), -1)
    assert (a - b).abs().max().item() < 1e-5


def test_smoothed_v_blocks_have_near_zero_mean():
    v = cpu_randn(1, 256, 2, 64, seed=7, dtype=torch.float32) + 5.0
    vc, _ = opre.smooth_v_per_block(v, block_s=64)
    assert vc.reshape(1, 4, 64, 2, 64).mean(2).abs().max().item() < 1e-5
