"""GPU quantisers / dequantisers: codes and scales bit-exact vs the CPU oracle
(reference quant_triton.py semantics)."""

import pytest
import torch

from conftest import cpu_randn
from oracle import quant as oq

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _inputs(shape, dtype, seed):
    x = cpu_randn(*shape, seed=seed, dtype=torch.float32, scale=2.0)
    x[..., 3] *= 20.0  # an outlier channel
    # signed zeros and values far below the E4M3 range: their codes are
    # +-0 with the sign of x (0x80 for a negative quotient)
    f = x.view(-1)
    f[::97] = -0.0
    f[1::101] = 0.0
    f[2::103] = -1e-30
    f[3::107] = 1e-30
    return x.to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d,block", [(64, 64), (128, 128), (128, 64), (64, 32)])
def test_fp8_block_quant_bit_exact(gpu, dtype, d, block):
    from low_bit_fake_quant import fp8_block_dequant, fp8_block_quant
    x = _inputs((2, 512, 3, d), dtype, seed=d + block)
    codes, sc = fp8_block_quant(x.to(gpu), block_s=block)
    rc, rs = oq.fp8_block_quant(x, block)
    assert codes.dtype == torch.float8_e4m3fn and codes.shape == x.shape
    assert torch.equal(codes.view(torch.uint8).cpu(), rc)
    assert torch.equal(sc.cpu(), rs)
    for odt in (torch.float32, torch.bfloat16):
        deq = fp8_block_dequant(codes, sc, block_s=block, dtype=odt)
        assert torch.equal(deq.cpu(), oq.fp8_block_dequant(rc, rs, block, dtype=odt))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [64, 128])
def test_fp8_channel_quant_bit_exact(gpu, dtype, d):
    from low_bit_fake_quant import fp8_per_channel_dequant, fp8_per_channel_quant
    x = _inputs((1, 1000, 2, d), dtype, seed=7 + d)
    codes, sc = fp8_per_channel_quant(x.to(gpu))
    rc, rs = oq.fp8_per_channel_quant(x)
    assert torch.equal(codes.view(torch.uint8).cpu(), rc)
    assert torch.equal(sc.cpu(), rs)
    deq = fp8_per_channel_dequant(codes, sc, dtype=torch.bfloat16)
    assert torch.equal(deq.cpu(), oq.fp8_per_channel_dequant(rc, rs, dtype=torch.bfloat16))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d,block_d", [(128, 32), (64, 32), (128, 64), (128, 16)])
def test_mxfp8_qk_quant_bit_exact(gpu, dtype, d, block_d):
    from low_bit_fake_quant import mxfp8_qk_dequant, mxfp8_qk_quant
    if block_d < 8:
        pytest.skip("block below 8 columns")
    x = _inputs((1, 300, 2, d), dtype, seed=11 + block_d)
    codes, sc = mxfp8_qk_quant(x.to(gpu), block_d=block_d)
    rc, rs = oq.mxfp8_qk_quant(x, block_d)
    assert torch.equal(codes.view(torch.uint8).cpu(), rc)
    assert torch.equal(sc.cpu(), rs)
    deq = mxfp8_qk_dequant(codes, sc, block_d=block_d)
    assert torch.equal(deq.cpu(), oq.mxfp8_qk_dequant(rc, rs, block_d))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d,block", [(128, 64), (64, 32), (128, 128)])
def test_mxfp8_v_quant_bit_exact(gpu, dtype, d, block):
    from low_bit_fake_quant import mxfp8_v_dequant, mxfp8_v_quant
    x = _inputs((2, 256, 2, d), dtype, seed=13 + block)
    codes, sc = mxfp8_v_quant(x.to(gpu), block_s=block)
    rc, rs = oq.mxfp8_v_quant(x, block)
    assert torch.equal(codes.view(torch.uint8).cpu(), rc)
    assert torch.equal(sc.cpu(), rs)
    deq = mxfp8_v_dequant(codes, sc, block_s=block, dtype=torch.float32)
    assert torch.equal(deq.cpu(), oq.mxfp8_v_dequant(rc, rs, block))


def test_zero_block_and_error_messages(gpu):
    from low_bit_fake_quant import fp8_block_quant, mxfp8_qk_quant
    x = torch.zeros(1, 128, 1, 64, dtype=torch.bfloat16, device=gpu)
    codes, sc = fp8_block_quant(x, block_s=128)
    rc, rs = oq.fp8_block_quant(x.cpu(), 128)
    assert torch.equal(sc.cpu(), rs) and int(codes.view(torch.uint8).max()) == 0
    with pytest.raises(ValueError, match="must be divisible by block_s"):
        fp8_block_quant(torch.zeros(1, 100, 1, 64, device=gpu), block_s=64)
    with pytest.raises(ValueError, match=r"shape\[-1\] must be 64 or 128"):
        mxfp8_qk_quant(torch.zeros(1, 64, 1, 32, device=gpu))


def test_non_finite_inputs_quantise_like_the_reference(gpu):
    """The reference clamps with tl.minimum(tl.maximum(x / sc, -448), 448) and
    takes amax with tl.max (quant_triton.py:47-49, 151-159, 240-244, 339-343),
    Triton's maximum / minimum without NaN propagation, which return the
    non-NaN operand (IEEE maxNum / minNum).  So a NaN element drops out of its
    block's amax and quantises to -448 (code 0xFE); every other code and every
    scale are those of the same input with the NaN read as 0.  (The CPU oracle
    uses torch's NaN-propagating clamp and amax, so it is not the reference
    here.)  +-inf: an fp8_block / channel scale becomes inf, inf / inf = NaN
    gives -448; the MX scales clamp their E8M0 exponent, so +-inf gives +-448."""
    from low_bit_fake_quant import fp8_block_quant, fp8_per_channel_quant, mxfp8_qk_quant, mxfp8_v_quant
    quants = {
        "fp8_block": (lambda t: fp8_block_quant(t, block_s=64), lambda t: oq.fp8_block_quant(t, 64)),
        "channel": (fp8_per_channel_quant, oq.fp8_per_channel_quant),
        "mx_qk": (lambda t: mxfp8_qk_quant(t, block_d=32), lambda t: oq.mxfp8_qk_quant(t, 32)),
        "mx_v": (lambda t: mxfp8_v_quant(t, block_s=64), lambda t: oq.mxfp8_v_quant(t, 64)),
    }
    x = _inputs((1, 128, 2, 64), torch.bfloat16, seed=77)
    pos = (0, 5, 1, 3)
    for name, (gq, cq) in quants.items():
        xn = x.clone()
        xn[pos] = float("nan")
        codes, sc = gq(xn.to(gpu))
        c = codes.view(torch.uint8).cpu()
        assert c[pos].item() == 0xFE, name
        x0 = x.clone()
        x0[pos] = 0.0
        rc, rs = cq(x0)
        rc = rc.clone()
        rc[pos] = 0xFE
        assert torch.equal(c, rc), name
        assert torch.equal(sc.cpu(), rs), name
        for val, code in ((float("inf"), 0x7E if name.startswith("mx") else 0xFE), (float("-inf"), 0xFE)):
            xi = x.clone()
            xi[pos] = val
            codes, sc = gq(xi.to(gpu))
            assert codes.view(torch.uint8).cpu()[pos].item() == code, (name, val)
            assert bool(torch.isfinite(sc.float().cpu()).all()) == name.startswith("mx"), (name, val)
