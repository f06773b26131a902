"""Pins the Hadamard oracle (reference hadamard.py:25-117) against the textbook
Sylvester matrix, orthonormality, logit preservation and the committed sign
fixture; also pins the E4M3 encoder against the committed bf16 code table."""

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


# ---- Hadamard (reference hadamard.py:25-117) ---------------------------------


def test_signs_match_golden_fixture():
    ref = np.load(os.path.join(GOLDEN, "hadamard_signs_h40_d128_seed0.npy"))
    assert np.array_equal(ohad.signs(40, 128, 0).numpy(), ref)
    assert set(np.unique(ref).tolist()) == {-1, 1}


@pytest.mark.parametrize("d", [64, 128])
def test_fwht_equals_sylvester_matrix_and_is_orthonormal(d):
    eye = torch.eye(d)
    rows = ohad.fwht_last_dim(eye, 1.0)
    h = torch.from_numpy(scipy.linalg.hadamard(d).astype(np.float32))
    assert torch.equal(rows, h)
    scaled = ohad.fwht_last_dim(eye, 1.0 / math.sqrt(d))
    assert torch.allclose(scaled @ scaled.T, eye, atol=1e-6)


def test_rotation_preserves_logits():
    q = cpu_randn(1, 64, 3, 128, seed=1, dtype=torch.float32)
    k = cpu_randn(1, 64, 3, 128, seed=2, dtype=torch.float32)
    qr, kr = ohad.apply_qk_hadamard(q, k, random_sign=True, seed=0)
    a = torch.einsum("bshd,bthd->bhst", q.double(), k.double())
    b = torch.einsum("bshd,bthd->bhst", qr.double(), kr.double())
    assert (a - b).abs().max().item() < 2e-4


def test_rotation_spreads_an_outlier_channel():
    x = torch.zeros(1, 1, 1, 128)
    x[..., 5] = 100.0
    r, _ = ohad.apply_qk_hadamard(x, x, random_sign=True, seed=0)
    assert torch.allclose(r.abs(), torch.full_like(r, 100.0 / math.sqrt(128)), rtol=1e-6)


# ---- E4M3 golden table -------------------------------------------------------


def test_e4m3_encoder_matches_golden_table():
    table = np.load(os.path.join(GOLDEN, "e4m3_bf16_codes.npy"))
    vals = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    finite = np.isfinite(vals)
    x = np.clip(vals[finite], -448.0, 448.0).astype(np.float32)
    assert np.array_equal(fp8.encode(x), table[finite])
