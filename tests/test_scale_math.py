"""CPU pin of the exponent identity the MX-P attention kernels use
(ceil_log2_div448 in csrc/lbfq_common.h): for positive normal fp32 r,
ceil(log2(fl32(r / 448))) equals exponent(r) - 8 + [mantissa(r) > 0.75],
checked against IEEE float32 division (numpy) over every mantissa of
several exponents."""

import numpy as np


def test_ceil_log2_div448_matches_ieee_division():
    mant = np.arange(1 << 23, dtype=np.uint32)
    for e in (-100, -14, -1, 0, 1, 7, 8, 9, 20, 100):
        bits = (np.uint32(e + 127) << np.uint32(23)) | mant
        r = bits.view(np.float32)
        q = (r / np.float32(448.0)).astype(np.float32)
        qb = q.view(np.uint32)
        ref = (qb >> 23).astype(np.int64) - 127 + ((qb & 0x7FFFFF) != 0)     # ceil(log2(q)), q normal
        got = (bits >> 23).astype(np.int64) - 127 - 8 + (mant > 0x600000)
        assert np.array_equal(ref, got), e
