"""Pins the k-means reorder oracle (reference kmeans.py:44-135; clustering per
this build's own Lloyd specification): C oracle == scalar restatement, labels
are nearest centroids, well-separated clusters are recovered, stable-sort
order / inverse round trip, K/V co-permutation invariance."""

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
