"""Pins the Hadamard, smoothing and k-means-reorder parts of the oracle by
independent checks (textbook matrices, exact rational means, brute force,
invariants) and the committed golden fixtures."""

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


# ---- k-means reorder (reference kmeans.py:44-135) ----------------------------


def test_kmeans_c_oracle_equals_scalar_restatement():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 96, 8, generator=g).numpy().astype(np.float32)
    lab, cent = okm.kmeans_labels(x, 4, 3, 123)
    for bh in range(2):
        lab_py, cent_py = okm.kmeans_labels_py(x[bh], 4, 3, 123, bh=bh)
        assert np.array_equal(lab[bh], lab_py)
        assert np.array_equal(cent[bh], cent_py)


def test_kmeans_labels_are_nearest_centroid():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 200, 16, generator=g).numpy().astype(np.float32)
    lab, cent = okm.kmeans_labels(x, 5, 0, 7)   # 0 iterations: assignment to the initial centroids
    d2 = ((x[0, :, None, :].astype(np.float64) - cent[0][None].astype(np.float64)) ** 2).sum(-1)
    best = d2.min(1)
    chosen = d2[np.arange(200), lab[0]]
    assert np.all(chosen <= best + 1e-4 * (1 + best))


def test_kmeans_separates_well_separated_clusters():
    g = torch.Generator().manual_seed(10)
    cent = torch.randn(4, 16, generator=g) * 20
    # tokens laid out cluster by cluster: the strided initialisation (one seed
    # token per S/k stretch) then starts one centroid in every cluster
    assign = torch.arange(256) // 64
    x = (cent[assign] + 0.01 * torch.randn(256, 16, generator=g)).numpy()[None].astype(np.float32)
    lab, _ = okm.kmeans_labels(x, 4, 10, 0)
    # same true cluster <=> same label
    same_true = assign[:, None] == assign[None, :]
    same_lab = torch.from_numpy(lab[0])[:, None] == torch.from_numpy(lab[0])[None, :]
    assert torch.equal(same_true, same_lab)


def test_reorder_is_stable_sort_with_inverse():
    labels = torch.tensor([[2, 0, 2, 1, 0, 1, 2, 0]])
    order, inverse = okm.reorder_from_labels(labels)
    assert order.tolist() == [[1, 4, 7, 3, 5, 0, 2, 6]]
    assert torch.equal(torch.gather(order, 1, inverse), torch.arange(8).unsqueeze(0))


def test_reorder_roundtrip_and_kv_copermutation_invariance():
    t = cpu_randn(1, 128, 2, 16, seed=11, dtype=torch.float32)
    v = cpu_randn(1, 128, 2, 16, seed=12, dtype=torch.float32)
    q = cpu_randn(1, 128, 2, 16, seed=13, dtype=torch.float32)
    res = okm.kmeans_reorder_tokens(t, n_clusters=8, max_iters=3, seed=1)
    back = okm.apply_kv_permutation(res["tensor_reordered"], res["inverse_order"])
    assert torch.equal(back, t)
    # attention over keys is invariant to a common permutation of K and V
    kp = okm.apply_kv_permutation(t, res["order"])
    vp = okm.apply_kv_permutation(v, res["order"])
    a = torch.softmax(torch.einsum("bshd,bthd->bhst", q, t), -1) @ v.permute(0, 2, 1, 3)
    b = torch.softmax(torch.einsum("bshd,bthd->bhst", q, kp), -1) @ vp.permute(0, 2, 1, 3)
    assert (a - b).abs().max().item() < 1e-5
