"""Pins of the probe oracle (``oracle/probe.py``) on the CPU.

* ``p_requant_rows`` against float64 softmax / logsumexp (closed forms of the
  reference probe, ``p_requant.py:12-41``), the exact E4M3 code of 2^offset at
  the row max, and saturation at 448.
* ``rowmax_counts`` on hand-built tile sequences whose six counters follow
  from the reference rules (``bench/count_rowmax_updates_triton.py:128-171``)
  by hand, and natural-units == log2-units on the same logits.
"""

import math

import numpy as np
import pytest
import torch

from oracle import fp8
from oracle import probe

LOG2E = 1.4426950408889634


def _scores(seed=0, shape=(2, 5, 37), scale=3.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


@pytest.mark.parametrize("off", [0, 8])
def test_p_requant_rows_closed_forms(off):
    x = _scores()
    sm = 0.125
    codes, row_sum, lse = probe.p_requant_rows(x, sm_scale=sm, p_max_offset=off)
    xd = x.double()
    e = torch.exp(sm * (xd - xd.amax(-1, keepdim=True))) * 2.0 ** off
    # lse is log-sum-exp of the scaled logits, independent of the offset
    assert torch.allclose(lse.double(), torch.logsumexp(sm * xd, dim=-1), atol=2e-6, rtol=0)
    assert torch.allclose(row_sum.double(), e.sum(-1), rtol=2e-6, atol=0)
    # the row max maps to exactly 2^offset
    am = x.argmax(-1, keepdim=True)
    assert (torch.gather(codes, -1, am) == int(fp8.encode(np.array([2.0 ** off], dtype=np.float32))[0])).all()
    # every code is the nearest E4M3 value of p (half an E4M3 step, 2^-4 relative, in the normal range)
    dec = torch.from_numpy(fp8.decode(codes.numpy())).double()
    normal = e >= 2.0 ** -6
    assert ((dec - e).abs()[normal] <= e[normal] * 2.0 ** -4 * 1.0001).all()
    assert ((dec - e).abs()[~normal] <= 2.0 ** -10 * 1.0001).all()


def test_p_requant_rows_saturates():
    x = _scores(seed=1)
    codes, _, _ = probe.p_requant_rows(x, sm_scale=0.125, p_max_offset=10)
    am = x.argmax(-1, keepdim=True)
    assert (torch.gather(codes, -1, am) == 0x7E).all()  # 1024 -> 448


def _rows(*tile_max_lists, block=4, fill=-1000.0):
    """(R, N) log2 scores whose tile t of row r has maximum tile_max_lists[r][t]."""
    n = block * len(tile_max_lists[0])
    s = torch.full((len(tile_max_lists), n), fill)
    for r, tms in enumerate(tile_max_lists):
        for t, v in enumerate(tms):
            s[r, t * block] = v
    return s


def test_online_rule_counts_by_hand():
    s = _rows([0, 5, 20, 10, 40], [3, 3, 3, 3, 3])
    c = probe.rowmax_counts(s, None, up=8, down=8, use_estimate=False, block_n=4, units="log2")
    # row 0: tiles 0 (first), 2 (+20), 4 (+20) update; row 1: tile 0 only
    assert c == {"updates": 4, "rescales": 2, "upward_updates": 4, "downward_updates": 0,
                 "rows_with_update": 2, "max_updates_per_row": 3}


def test_estimated_rule_counts_by_hand():
    # row 0: estimate far above, no mass yet -> one downward jump to the tile max, no rescale
    # row 1: estimate 0; +20 and +30 exceed up=16 (+5 does not) -> two upward updates with rescale
    # row 2: estimate 10 is within down=16 of the maxima -> no update
    s = _rows([0, 0, 0, 0], [0, 20, 25, 50], [0, 1, 2, 3])
    m0 = torch.tensor([100.0, 0.0, 10.0])
    c = probe.rowmax_counts(s, m0, up=16, down=16, use_estimate=True, block_n=4, units="log2")
    assert c == {"updates": 3, "rescales": 2, "upward_updates": 2, "downward_updates": 1,
                 "rows_with_update": 2, "max_updates_per_row": 2}


def test_units_are_equivalent():
    g = torch.Generator().manual_seed(3)
    u2 = torch.randn(64, 256, generator=g) * 12.0
    m0 = u2.amax(1) + torch.randn(64, generator=g) * 20.0
    for est in (False, True):
        a = probe.rowmax_counts(u2, m0, up=8.0, down=16.0, use_estimate=est, units="log2")
        b = probe.rowmax_counts((u2.double() / LOG2E).float(), (m0.double() / LOG2E).float(), up=8.0, down=16.0,
                                use_estimate=est, units="natural")
        assert a == b
        assert a["updates"] > 0
