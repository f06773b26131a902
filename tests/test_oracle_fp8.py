"""Pins the oracle's E4M3FN codec against torch.float8_e4m3fn (CPU)."""

import numpy as np
import torch

from oracle import fp8


def _torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_table_matches_torch():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    d = fp8.DECODE
    same = (d == ref) | (np.isnan(d) & np.isnan(ref))
    assert same.all()


def test_encode_all_bf16_patterns_with_low_fills():
    hi = np.arange(65536, dtype=np.uint32) << 16
    for lo in (0x0000, 0x8000, 0x7FFF, 0x0001, 0xFFFF, 0x4321):
        x = (hi | lo).view(np.float32)
        x = np.clip(x, -448.0, 448.0)
        x = x[~np.isnan(x)]
        assert np.array_equal(fp8.encode(x), _torch_codes(x)), hex(lo)


def test_encode_midpoints_and_neighbours():
    vals = np.unique(np.abs(fp8.DECODE[~np.isnan(fp8.DECODE)]).astype(np.float64))
    mids = (vals[:-1] + vals[1:]) / 2.0
    pts = np.concatenate([vals, mids]).astype(np.float32)
    up = np.nextafter(pts, np.float32(np.inf))
    dn = np.nextafter(pts, np.float32(-np.inf))
    x = np.concatenate([pts, up, dn, -pts, -up, -dn])
    x = np.clip(x, -448.0, 448.0)
    assert np.array_equal(fp8.encode(x), _torch_codes(x))


def test_encode_random_fp32():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1_000_000) * rng.choice([1e-4, 1e-2, 1, 30, 300], 1_000_000)).astype(np.float32)
    x = np.clip(x, -448, 448)
    assert np.array_equal(fp8.encode(x), _torch_codes(x))


def test_saturation_and_nan():
    assert fp8.encode(np.float32(1e6)).item() == 0x7E
    assert fp8.encode(np.float32(-1e30)).item() == 0xFE
    assert fp8.encode(np.float32(np.inf)).item() == 0x7E
    assert fp8.encode(np.float32(np.nan)).item() & 0x7F == 0x7F
    # round-to-nearest-even at the top of the range: 448 < x < 464 -> 448
    assert fp8.encode(np.float32(460.0)).item() == 0x7E


def test_round_trip_exact_on_representable():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    vals = fp8.decode(codes)
    back = fp8.encode(vals)
    # +0 and -0 keep their codes; every finite value round-trips
    assert np.array_equal(back, codes)
