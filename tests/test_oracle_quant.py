"""Pins the quantiser oracle (reference quant_triton.py) by independent checks."""

import fractions
import math

import numpy as np
import pytest
import torch

from conftest import cpu_randn
from oracle import fp8
from oracle import quant as oq

FINITE_VALUES = np.array(sorted(set(fp8.DECODE[~np.isnan(fp8.DECODE)].tolist())), dtype=np.float64)


def _nearest_code_value(y: np.ndarray) -> np.ndarray:
    """Brute force: nearest E4M3 value to y (clamped), ties to the even code."""
    y = np.clip(y.astype(np.float64), -448, 448)
    dist = np.abs(y[:, None] - FINITE_VALUES[None, :])
    best = dist.min(axis=1, keepdims=True)
    cand = dist == best
    out = np.empty(len(y))
    for i in range(len(y)):
        vals = FINITE_VALUES[cand[i]]
        if len(vals) == 1:
            out[i] = vals[0]
        else:  # tie: pick the one whose code mantissa is even
            codes = fp8.encode(vals.astype(np.float32))
            out[i] = vals[(codes & 1) == 0][0]
    return out


def test_fp8_block_codes_are_nearest_and_amax_maps_to_448():
    x = cpu_randn(1, 256, 2, 64, seed=1, scale=3.0)
    codes, sc = oq.fp8_block_quant(x, 64)
    xf = x.float().reshape(1, 4, 64, 2, 64)
    amax = xf.abs().amax(dim=(2, 4))
    assert torch.equal(sc, (amax / 448.0).float())  # fp32 division of fp32 values
    y = (xf / sc[:, :, None, :, None]).reshape(-1).numpy()
    got = fp8.decode(codes.reshape(-1).numpy()).astype(np.float64)
    assert np.array_equal(got, _nearest_code_value(y))
    # the element with the largest magnitude quantises to +-448
    dec = fp8.decode(codes.numpy()).reshape(1, 4, 64, 2, 64)
    assert np.allclose(np.abs(dec).max(axis=(2, 4)), 448.0)


def test_fp8_block_zero_block_floor():
    x = torch.zeros(1, 128, 1, 64, dtype=torch.bfloat16)
    codes, sc = oq.fp8_block_quant(x, 128)
    assert sc.item() == np.float32(np.float32(1e-4) / np.float32(448.0))
    assert int(codes.max()) == 0


def test_channel_scale_is_column_amax():
    x = cpu_randn(2, 96, 3, 64, seed=2)
    codes, sc = oq.fp8_per_channel_quant(x)
    assert torch.equal(sc, x.float().abs().amax(dim=1).clamp_min(float(np.float32(1e-4))) / 448.0)
    deq = oq.fp8_per_channel_dequant(codes, sc)
    rel = ((deq - x.float()).abs() / sc[:, None]).max().item()
    assert rel <= 16.0 * (1 + 1e-5)  # half an E4M3 ulp at the top binade (32), in code units


def test_ceil_log2_exact_against_fractions():
    rng = np.random.default_rng(3)
    r = np.concatenate([
        (rng.random(2000) * 100).astype(np.float32),
        np.ldexp(np.float32(1.0), rng.integers(-30, 30, 200)).astype(np.float32),
    ])
    r = r[r > 0]
    r = np.concatenate([r, np.nextafter(r, np.float32(np.inf)), np.nextafter(r, np.float32(0))])
    got = oq.ceil_log2_exact(r)
    for v, e in zip(r.tolist(), got.tolist()):
        f = fractions.Fraction(v)
        assert fractions.Fraction(2) ** (e - 1) < f <= fractions.Fraction(2) ** e


@pytest.mark.parametrize("block_d", [32, 64])
def test_mx_qk_scales_are_pow2_and_fill_range(block_d):
    x = cpu_randn(1, 64, 2, 128, seed=4, scale=5.0)
    codes, sc = oq.mxfp8_qk_quant(x, block_d)
    m, e = np.frexp(sc.numpy())
    assert np.all(m == 0.5)  # exact powers of two
    xb = x.float().reshape(1, 64, 2, 128 // block_d, block_d).abs().amax(-1)
    ratio = (xb / sc).numpy()
    assert np.all(ratio <= 448.0) and np.all(ratio > 224.0)
    deq = oq.mxfp8_qk_dequant(codes, sc, block_d)
    y = (x.float().reshape(1, 64, 2, -1, block_d) / sc[..., None]).reshape(-1).numpy()
    assert np.array_equal((deq.reshape(1, 64, 2, -1, block_d) / sc[..., None]).reshape(-1).numpy(),
                          _nearest_code_value(y).astype(np.float32))


def test_mx_v_scale_per_block_column():
    x = cpu_randn(1, 128, 2, 64, seed=5, scale=2.0)
    codes, sc = oq.mxfp8_v_quant(x, 64)
    assert sc.shape == (1, 2, 2, 64)
    amax = x.float().reshape(1, 2, 64, 2, 64).abs().amax(2)
    for a, s in zip(amax.flatten().tolist(), sc.flatten().tolist()):
        e = math.ceil(math.log2(max(a, 1e-4) / 448.0))
        assert s == 2.0 ** e or abs(math.log2(max(a, 1e-4) / 448.0) - round(math.log2(max(a, 1e-4) / 448.0))) < 1e-9


def test_block_dequant_matches_definition():
    x = cpu_randn(1, 128, 2, 64, seed=6)
    codes, sc = oq.fp8_block_quant(x, 64)
    deq = oq.fp8_block_dequant(codes, sc, 64, dtype=torch.float32)
    ref = torch.from_numpy(fp8.decode(codes.numpy())).reshape(1, 2, 64, 2, 64) * sc[:, :, None, :, None]
    assert torch.equal(deq, ref.reshape(1, 128, 2, 64))
