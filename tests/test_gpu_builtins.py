"""GPU unit tests of the gfx950 builtins the kernels rely on: the hardware
FP32->E4M3 converter (v_cvt_pk_fp8_f32) and the lane layout / block scaling
of v_mfma[_scale]_f32_32x32x64_f8f6f4."""

import numpy as np
import pytest
import torch

from oracle import fp8

pytestmark = pytest.mark.gpu


def _lib():
    from low_bit_fake_quant import _lib as L
    return L, L.load()


def test_hw_cvt_matches_rne_encoder(gpu):
    L, lib = _lib()
    vals = np.unique(np.abs(fp8.DECODE[~np.isnan(fp8.DECODE)]).astype(np.float64))
    mids = ((vals[:-1] + vals[1:]) / 2.0).astype(np.float32)
    rng = np.random.default_rng(0)
    rnd = (rng.random(200_000) * 448.0).astype(np.float32)
    tiny = (rng.random(50_000) * 2.0 ** -5).astype(np.float32)
    base = np.concatenate([vals.astype(np.float32), mids, np.nextafter(mids, np.float32(0)),
                           np.nextafter(mids, np.float32(448)), rnd, tiny])
    x = np.clip(np.concatenate([base, -base]), -448, 448).astype(np.float32)
    if len(x) % 2:
        x = x[:-1]
    xt = torch.from_numpy(x).to(gpu)
    out = torch.empty(len(x), dtype=torch.uint8, device=gpu)
    L.check(lib.lbfq_selftest_cvt_fp8(xt.data_ptr(), len(x), out.data_ptr(), L.stream_handle()), "cvt")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = fp8.encode(x)
    bad = np.nonzero(got != ref)[0]
    assert len(bad) == 0, f"{len(bad)} mismatches, e.g. x={x[bad[:5]]} hw={got[bad[:5]]} ref={ref[bad[:5]]}"


def _rand_codes(rng, shape):
    c = rng.integers(0, 256, size=shape, dtype=np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x38  # no NaN codes
    return c


@pytest.mark.parametrize("scaled", [False, True])
def test_mfma_32x32x64_layout_and_scales(gpu, scaled):
    L, lib = _lib()
    rng = np.random.default_rng(1 if scaled else 2)
    A = _rand_codes(rng, (32, 64))
    B = _rand_codes(rng, (64, 32))
    Af = fp8.decode(A).astype(np.float64)
    Bf = fp8.decode(B).astype(np.float64)
    if scaled:
        sa = rng.integers(120, 135, size=(32, 2)).astype(np.uint8)
        sb = rng.integers(120, 135, size=(32, 2)).astype(np.uint8)
        ref = np.zeros((32, 32))
        for blk in range(2):
            ks = slice(32 * blk, 32 * blk + 32)
            fa = np.ldexp(1.0, sa[:, blk].astype(int) - 127)[:, None]
            fb = np.ldexp(1.0, sb[:, blk].astype(int) - 127)[None, :]
            ref += (Af[:, ks] @ Bf[ks, :]) * fa * fb
    else:
        ref = Af @ Bf
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    a_d, b_d = t(A), t(B)
    sa_d = t(sa) if scaled else None
    sb_d = t(sb) if scaled else None
    c = torch.empty((32, 32), dtype=torch.float32, device=gpu)
    L.check(lib.lbfq_selftest_mfma(a_d.data_ptr(), b_d.data_ptr(), L.ptr(sa_d), L.ptr(sb_d), c.data_ptr(),
                                   L.stream_handle()), "mfma")
    torch.cuda.synchronize()
    got = c.cpu().numpy().astype(np.float64)
    # The FP8 MFMA accumulates with reduced internal precision (not exact fp32):
    # measured relative error ~1e-4 of the largest partial sums.
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 5e-4, f"relative error {err:.2e}"
    # the layout itself must be right: every element close to its own reference
    assert np.corrcoef(got.ravel(), ref.ravel())[0, 1] > 0.999999


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 1 << 22])
def test_hbm_stream_probe_moves_exactly_the_bytes(gpu, nbytes):
    """lbfq_hbm_stream (the prepass ceiling probe): the copy mode copies the
    bytes exactly, the write mode writes word i's index into its first dword
    and nothing past the end, the read mode writes nothing; partial last
    chunks included."""
    from low_bit_fake_quant import _lib
    lib = _lib.load()
    st = _lib.stream_handle(gpu)
    n16 = nbytes // 16
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n16 + 4, 4), dtype=torch.int32, device=gpu)
    sink = torch.zeros(256, dtype=torch.int32, device=gpu)
    for mode in (0, 1, 2):
        dst = torch.full((n16 + 4, 4), -7, dtype=torch.int32, device=gpu)
        _lib.check(lib.lbfq_hbm_stream(mode, src.data_ptr(), dst.data_ptr(), nbytes, 64, sink.data_ptr(), st),
                   "lbfq_hbm_stream")
        torch.cuda.synchronize()
        want = torch.full_like(dst, -7)
        if mode == 1:
            want[:n16] = 0
            want[:n16, 0] = torch.arange(n16, dtype=torch.int32, device=gpu)
        elif mode == 2:
            want[:n16] = src[:n16]
        assert torch.equal(dst, want), mode
    with pytest.raises(ValueError, match="multiple of 16"):
        _lib.check(lib.lbfq_hbm_stream(2, src.data_ptr(), dst.data_ptr(), 24, 64, sink.data_ptr(), st),
                   "lbfq_hbm_stream")


@pytest.mark.parametrize("op", [0, 4, 7, 8])
def test_issue_probe_records_every_wave(gpu, op):
    """lbfq_issue_probe (the attention floor measurement): at 2 waves per
    SIMD every wave records a positive s_memtime span and a SIMD id, each of
    the 4 SIMDs holds 2 waves, and the per-instruction cost is plausible
    (at least 1 cycle, an MFMA at least the 32x32x64 FP8 rate of 64 cycles
    less 10%)."""
    from low_bit_fake_quant import _lib
    lib = _lib.load()
    rec = torch.zeros(8 * 3, dtype=torch.int64, device=gpu)
    sink = torch.zeros(512, dtype=torch.float32, device=gpu)
    iters = 200
    _lib.check(lib.lbfq_issue_probe(op, 2, iters, rec.data_ptr(), sink.data_ptr(), _lib.stream_handle(gpu)),
               "lbfq_issue_probe")
    torch.cuda.synchronize()
    r = rec.view(8, 3).cpu()
    assert (r[:, 1] > r[:, 0]).all()
    assert sorted(r[:, 2].tolist()) == [0, 0, 1, 1, 2, 2, 3, 3]
    per_iter = {0: 16, 4: 16, 7: 8, 8: 1}[op]
    cost = (r[:, 1].max() - r[:, 0].min()).item() / (8 * iters * per_iter) * 4
    assert cost >= (57.6 if op == 7 else 1.0)
    with pytest.raises(ValueError, match="1 or 2 waves"):
        _lib.check(lib.lbfq_issue_probe(0, 3, 1, rec.data_ptr(), sink.data_ptr(), _lib.stream_handle(gpu)), "x")
