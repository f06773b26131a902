"""Pins of the BLASST simulator oracle (``oracle/blasst_sim.py``) and of the
package's predicate / reorder helpers, on the CPU.

The oracle's rungs are checked against float64 softmax attention (exact rung
on the raw operands, online rung on the dequantised operands), the static /
skip relations the reference states (skip at threshold 0 == static, bitwise;
skip rate monotone; the empty-tile safeguard), the tile keep masks against a
brute-force per-row evaluation of the predicate, and the per-head quant
against ``torch.float8_e4m3fn``.  The helper tests restate the reference's
own unit cases (``tests/test_blasst_skip.py:236-275, 336-352, 408-435,
437-478``).
"""

import math

import pytest
import torch

from conftest import cpu_randn
from oracle import blasst_sim as osim

from low_bit_fake_quant import blasst_skip as bs


def _qkv(s=256, h=2, d=64, seed=0):
    return (cpu_randn(1, s, h, d, seed=seed), cpu_randn(1, s, h, d, seed=seed + 1),
            cpu_randn(1, s, h, d, seed=seed + 2))


def _attn64(q, k, v):
    qf, kf, vf = (t[0].double().permute(1, 0, 2) for t in (q, k, v))
    p = torch.softmax(qf @ kf.transpose(1, 2) / math.sqrt(q.shape[-1]), dim=-1)
    return (p @ vf).permute(1, 0, 2)


def _close(a, b, cos_min, rel):
    a, b = a.double().flatten(), b.double().flatten()
    cos = float(a @ b / (a.norm() * b.norm()))
    rr = float((a - b).norm() / b.norm())
    assert cos >= cos_min and rr <= rel, (cos, rr)


def test_rungs_against_float64_attention():
    q, k, v = _qkv()
    r = osim.simulate(q, k, v, skip_thresholds=[], mm_dtype=torch.float32)
    _close(r["bf16_ref"], _attn64(q, k, v), 0.999999, 1e-5)
    deq = [osim.head_quant(t[0])[0].unsqueeze(0) for t in (q, k, v)]
    _close(r["fp8_qkv"], _attn64(*deq), 0.999999, 1e-5)
    # static P differs from the online rung only by the E4M3 rounding of P
    _close(r["fp8_static_p"], r["fp8_qkv"], 0.999, 5e-2)
    rb = osim.simulate(q, k, v, skip_thresholds=[], mm_dtype=torch.bfloat16)
    _close(rb["bf16_ref"], _attn64(q, k, v), 0.99999, 5e-3)


def test_skip_zero_is_static_and_rate_is_monotone():
    torch.manual_seed(3)
    q, k, v = _qkv(s=512, seed=5)
    k = k.clone()
    k[:, :128] *= 8.0
    k[:, 128:] *= 0.02
    r = osim.simulate(q, k, v, skip_thresholds=[0.0, 0.1, 0.9])
    assert torch.equal(r["skip"][0.0], r["fp8_static_p"])
    assert r["skip_rate"][0.0] == 0.0
    assert r["skip_rate"][0.0] <= r["skip_rate"][0.1] <= r["skip_rate"][0.9]
    assert r["skip_rate"][0.9] > 0.0
    assert (r["dropped"][0.0] == 0).all() and (r["dropped"][0.9] >= 0).all()


def test_empty_tile_safeguard_keeps_the_largest_block():
    q, k, v = _qkv(s=512, seed=9)
    # log(2) > 0 drops every block (margins are <= 0): each tile keeps exactly one
    r = osim.simulate(q, k, v, skip_thresholds=[2.0, 1.0])
    keep = r["keep"][2.0]
    assert (keep.sum(-1) == 1).all()
    assert r["force"][2.0] == keep.shape[0] * keep.shape[1]
    assert r["force"][1.0] == 0  # block 0 always has margin 0
    # the kept block is the one of largest max-over-rows block max (brute force)
    qd, kd = (osim.head_quant(t[0])[0].to(torch.bfloat16).float().permute(1, 0, 2) for t in (q, k))
    sc = qd @ kd.transpose(1, 2) / 8.0
    h, s, _ = sc.shape
    bm = sc.view(h, s // 128, 128, s // 128, 128).amax(-1).amax(2)          # (h, tiles, blocks)
    assert torch.equal(keep.float().argmax(-1), bm.argmax(-1))
    assert torch.isfinite(r["skip"][2.0]).all()


def test_tile_keep_masks_brute_force():
    q, k, v = _qkv(s=384, seed=21)
    th = 0.05
    r = osim.simulate(q, k, v, skip_thresholds=[th])
    qd, kd = (osim.head_quant(t[0])[0].to(torch.bfloat16).float().permute(1, 0, 2) for t in (q, k))
    sc = (qd @ kd.transpose(1, 2)) * torch.tensor(1 / 8.0)
    h, s, _ = sc.shape
    nb = s // 128
    for hh in range(h):
        for mt in range(nb):
            for j in range(nb):
                keep = False
                for row in range(mt * 128, (mt + 1) * 128):
                    bms = [float(sc[hh, row, b * 128:(b + 1) * 128].max()) for b in range(j + 1)]
                    if bms[j] - max(bms) >= math.log(th):
                        keep = True
                        break
                assert bool(r["keep"][th][hh, mt, j]) == keep, (hh, mt, j)


def test_head_quant_matches_torch_cast():
    x = cpu_randn(256, 3, 64, seed=4, dtype=torch.float32) * 7.0
    deq, scale, st = osim.head_quant(x)
    sc = (x.abs().amax(dim=(0, 2)) / 448.0).clamp_min(torch.finfo(torch.float32).tiny).view(1, -1, 1)
    ref = (x / sc).to(torch.float8_e4m3fn).float() * sc
    assert torch.equal(deq, ref) and torch.equal(scale.view(1, -1, 1), sc)
    assert st["saturation_rate"] < 1e-4


# ---- helper semantics (the reference's unit cases) ---------------------------------------


def test_keep_mask_uses_running_not_final_max():
    block_max = torch.tensor([[1.0, 5.0, 3.0]])
    logt = math.log(0.1)
    assert bs.blasst_keep_mask(block_max, logt).tolist() == [[True, True, True]]
    final = (block_max - block_max.amax(-1, keepdim=True)) >= logt
    assert final.tolist() == [[False, True, True]]


def test_tile_keep_mask_is_all_rows_reduction():
    logt = math.log(0.1)
    bm = torch.tensor([[0.0, 0.0], [5.0, 0.0]]).unsqueeze(0)
    assert bs.blasst_tile_keep_mask(bm, logt).tolist() == [[True, True]]
    bm2 = torch.tensor([[5.0, 0.0], [5.0, 0.0]]).unsqueeze(0)
    assert bs.blasst_tile_keep_mask(bm2, logt).tolist() == [[True, False]]


def test_running_row_max_is_cummax():
    assert bs.running_row_max(torch.tensor([[2.0, 1.0, 4.0, 3.0]])).tolist() == [[2.0, 2.0, 4.0, 4.0]]


def test_static_p_quant_rule():
    p = torch.linspace(0, 1, 257)
    manual = (p * 256.0).to(torch.float8_e4m3fn).to(torch.float32) / 256.0
    assert torch.equal(bs.static_p_quant(p), manual)
    deq, sat, uf, sq, n = bs.static_p_quant_with_stats(p)
    assert torch.equal(deq, manual) and sat == 0 and n == 257
    assert uf == int(((manual == 0) & (p != 0)).sum())


def test_reorder_block_and_permutation():
    t, h, w = 20, 48, 72
    block = bs.choose_local_block(t, h, w)
    assert block[0] * block[1] * block[2] == 128
    perm = bs.space_time_reorder_index(t, h, w, block=block)
    assert not torch.equal(perm, torch.arange(t * h * w))
    assert sorted(perm.tolist()) == list(range(t * h * w))
    assert (perm[:128] // (h * w)).unique().numel() == block[0]
    # each block is one (bt, bh, bw) neighbourhood of the grid
    tt, hh, ww = perm[:128] // (h * w), (perm[:128] // w) % h, perm[:128] % w
    assert (tt.max() - tt.min() + 1, hh.max() - hh.min() + 1, ww.max() - ww.min() + 1) == block


def test_reorder_native_axis_order_and_roundtrip():
    t, h, w = 4, 8, 8
    perm = bs.space_time_reorder_index(t, h, w)
    inv = bs.invert_permutation(perm)
    x = torch.randn(1, t * h * w, 2, 16)
    assert torch.equal(bs.apply_token_permutation(bs.apply_token_permutation(x, perm), inv), x)
    # a (w, h, t) native order visits the same neighbourhoods through other indices
    p2 = bs.space_time_reorder_index(t, h, w, native_axis_order=("w", "h", "t"))
    assert sorted(p2.tolist()) == list(range(t * h * w)) and not torch.equal(p2, perm)
    with pytest.raises(ValueError):
        bs.choose_local_block(3, 5, 7)


def test_guards():
    bs.guard_no_full_matrix((8, 128, 4096), 4096)
    with pytest.raises(bs.FullMatrixAllocationError):
        bs.guard_no_full_matrix((8, 4096, 4096), 4096)
    from torch.nn.attention import SDPBackend
    assert SDPBackend.MATH in bs.select_sdpa_backends(512, force_math_backend=False, allow_math_fallback=True)
    big = bs.select_sdpa_backends(bs.MATH_BACKEND_SEQLEN_LIMIT, force_math_backend=False, allow_math_fallback=True)
    assert SDPBackend.MATH not in big and SDPBackend.FLASH_ATTENTION in big
    with pytest.raises(bs.FullMatrixAllocationError):
        bs.select_sdpa_backends(bs.MATH_BACKEND_SEQLEN_LIMIT, force_math_backend=True, allow_math_fallback=False)
    assert bs.select_sdpa_backends(256, force_math_backend=True, allow_math_fallback=False) == [SDPBackend.MATH]
