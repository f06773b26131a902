"""Degenerate inputs through the whole path, for the five benchmark recipes
(P requantisation with elementwise / dynamic / MX P, BLASST, and the SDPA path
with and without Q smoothing):

* all-zero Q, K and V: every scale at its floor, every score 0, V's smoothing
  means 0 -- the output is 0 (reference: quant_triton.py's zero-block floor,
  attention.py's smoothing);
* keys that are all equal: after K smoothing K_s = 0, without it every score
  of a query is the same -- the softmax is uniform and the output is the mean
  of the dequantised V;
* very peaked scores (Q scaled by 40): the dynamic P scale, the row-max
  estimate and BLASST see rows dominated by a few keys.

Each output is finite and agrees with the CPU oracle of the reference path
(zero and equal-key inputs within 1e-2 element-wise; peaked inputs through the
same checks as the random-input parity tests)."""

import dataclasses

import pytest
import torch

import parity
from conftest import cosine, max_abs
from oracle import pipeline as opipe
from test_gpu_attention import check_parity

pytestmark = pytest.mark.gpu

H, S, D = 2, 512, 128


def _recipes():
    from low_bit_fake_quant.wan import workloads
    w = workloads()
    return {
        "c0_sdpa": w[0].cfg,
        "c1_elementwise": w[1].cfg,
        "c2_dynamic_qmk": w[2].cfg,
        "c3_mx_vsmooth": w[3].cfg,
        "c4_blasst": w[4].cfg,
        "c2_sdpa_qm": dataclasses.replace(w[2].cfg, p_requant=False),
    }


RECIPES = sorted(_recipes())


def _inputs(case, seed=0):
    g = torch.Generator().manual_seed(seed)
    if case == "zeros":
        z = torch.zeros(1, S, H, D, dtype=torch.bfloat16)
        return z, z.clone(), z.clone()
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, S, H, D, generator=g)
    v = torch.randn(1, S, H, D, generator=g)
    if case == "equal_keys":
        k = k[:, :1].expand(1, S, H, D).contiguous()
    elif case == "peaked":
        q = q * 40.0
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


@pytest.mark.parametrize("case", ["zeros", "equal_keys", "peaked"])
@pytest.mark.parametrize("name", RECIPES)
def test_degenerate_inputs_match_oracle(gpu, name, case):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _recipes()[name]
    q, k, v = _inputs(case, seed=len(name))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    assert out.shape == q.shape and torch.isfinite(out.float()).all(), f"{name}/{case}: non-finite output"
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    assert torch.isfinite(ref.float()).all(), f"{name}/{case}: the oracle is not finite"
    if case == "zeros":
        assert out.float().abs().max().item() == 0.0, f"{name}: zero inputs give a non-zero output"
        assert ref.float().abs().max().item() == 0.0
        return
    if case == "equal_keys":
        # a uniform softmax: every row is the mean of the dequantised V rows
        m = max_abs(out, ref)
        assert m <= parity.MAXABS, f"{name}/equal_keys: max|diff| {m:.3e} against the oracle"
        return
    if cfg.p_requant:
        check_parity(out, q, k, v, cfg, label=f"{name}/peaked", dev=gpu)
    else:
        # the SDPA path runs on operands bit-equal to the oracle's: only fp32
        # accumulation order separates the two
        c, m = cosine(out, ref), max_abs(out, ref)
        assert c >= parity.COS_MIN and m <= parity.MAXABS, f"{name}/peaked: cos {c:.7f} max|diff| {m:.3e}"
