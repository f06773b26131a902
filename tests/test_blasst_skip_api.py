"""CPU behaviours of the BLASST simulator's helper API (``blasst_skip``) that
the reference's own test suite asserts (tests/test_blasst_skip.py:236-275,
336-352, 408-416, 424-452, 473-480): the keep masks use the running row max
and reduce over all rows of a tile, the space-time reorder is a genuine local
permutation, the static P rule, and the full-matrix / SDPA-backend guards.
(The GPU behaviours of the same file are in test_gpu_blasst_sim.py and
test_gpu_reference_behaviours.py.)"""

import math

import pytest
import torch
from torch.nn.attention import SDPBackend

from low_bit_fake_quant.blasst_skip import (
    MATH_BACKEND_SEQLEN_LIMIT,
    FullMatrixAllocationError,
    apply_token_permutation,
    blasst_keep_mask,
    blasst_tile_keep_mask,
    choose_local_block,
    guard_no_full_matrix,
    invert_permutation,
    running_row_max,
    select_sdpa_backends,
    space_time_reorder_index,
    static_p_quant,
)

LOG_T = math.log(0.1)


def test_keep_mask_is_against_the_running_max():
    bm = torch.tensor([[1.0, 5.0, 3.0]])
    # running max 1, 5, 5: margins 0, 0, -2, all above log 0.1
    assert blasst_keep_mask(bm, LOG_T).tolist() == [[True, True, True]]
    # against the final max (5 everywhere) the first block would go
    assert ((bm - bm.amax(-1, keepdim=True)) >= LOG_T).tolist() == [[False, True, True]]


def test_tile_keep_mask_keeps_a_block_any_row_needs():
    one_row_needs = torch.tensor([[[0.0, 0.0], [5.0, 0.0]]])
    assert blasst_tile_keep_mask(one_row_needs, LOG_T).tolist() == [[True, True]]
    no_row_needs = torch.tensor([[[5.0, 0.0], [5.0, 0.0]]])
    assert blasst_tile_keep_mask(no_row_needs, LOG_T).tolist() == [[True, False]]


def test_running_row_max_is_a_cumulative_max():
    assert running_row_max(torch.tensor([[2.0, 1.0, 4.0, 3.0]])).tolist() == [[2.0, 2.0, 4.0, 4.0]]


def test_space_time_reorder_is_a_local_permutation():
    t, h, w = 20, 48, 72
    blk = choose_local_block(t, h, w)
    assert blk[0] * blk[1] * blk[2] == 128
    perm = space_time_reorder_index(t, h, w, block=blk)
    assert not torch.equal(perm, torch.arange(t * h * w))
    assert torch.equal(torch.sort(perm).values, torch.arange(t * h * w))
    # the first 128-token block spans blk[0] frames
    assert (perm[:128] // (h * w)).unique().numel() == blk[0]


def test_token_permutation_round_trip():
    t, h, w = 4, 8, 8
    perm = space_time_reorder_index(t, h, w)
    x = torch.randn(1, t * h * w, 2, 16, generator=torch.Generator().manual_seed(0))
    assert torch.equal(apply_token_permutation(apply_token_permutation(x, perm), invert_permutation(perm)), x)
    assert torch.equal(torch.sort(perm).values, torch.arange(t * h * w))


def test_static_p_quant_rule():
    p = torch.linspace(0, 1, 257)
    want = (p * 256.0).to(torch.float8_e4m3fn).float() / 256.0
    got = static_p_quant(p)
    assert torch.equal(got, want) and got.max() <= 1.5


def test_sdpa_backend_guards():
    assert SDPBackend.MATH in select_sdpa_backends(512, force_math_backend=False, allow_math_fallback=True)
    big = select_sdpa_backends(MATH_BACKEND_SEQLEN_LIMIT, force_math_backend=False, allow_math_fallback=True)
    assert SDPBackend.MATH not in big and SDPBackend.FLASH_ATTENTION in big
    with pytest.raises(FullMatrixAllocationError):
        select_sdpa_backends(MATH_BACKEND_SEQLEN_LIMIT, force_math_backend=True, allow_math_fallback=False)
    assert select_sdpa_backends(256, force_math_backend=True, allow_math_fallback=False) == [SDPBackend.MATH]


def test_full_matrix_guard():
    guard_no_full_matrix((8, 128, 4096), 4096)
    with pytest.raises(FullMatrixAllocationError):
        guard_no_full_matrix((8, 4096, 4096), 4096)
