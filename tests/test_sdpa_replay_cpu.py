"""Pins ``parity.sdpa_replay``, the element-wise check of the SDPA path's output
(reference attention.py:288-319), on the CPU: an fp32 evaluation of the
reference's formulas -- the arithmetic the GPU kernel performs, up to
summation order -- passes it, and outputs carrying a planted mistake (a wrong
softmax scale, two keys' V rows swapped, the qm group of the next rows, a
missing rounding of the main score, one element moved by three ulps) fail it.
"""

import math
import types

import torch

import parity

LOG2E = 1.4426950408889634


def _operands(seed, s=200, pitch=256, h=2, d=64, groups=None, q_group=64, dt=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.zeros(1, h, pitch, d)
    k = torch.zeros(1, h, pitch, d)
    v_t = torch.zeros(1, h, d, pitch)
    q[:, :, :s] = torch.randn(1, h, s, d, generator=g)
    k[:, :, :s] = torch.randn(1, h, s, d, generator=g) * 1.5
    v_t[..., :s] = torch.randn(1, h, d, s, generator=g)
    bias = None
    if groups:
        bias = torch.zeros(1, h, groups, pitch)
        bias[..., :s] = torch.randn(1, h, groups, s, generator=g) * 2.0
    return types.SimpleNamespace(b=1, s=s, h=h, d=d, P=pitch, q=q.to(dt), k=k.to(dt), v_t=v_t.to(dt), bias=bias,
                                 q_group=q_group, out_row_map=None)


def _fp32_attention(ops, sm, *, scale=1.0, swap_keys=None, group_shift=0, round_main=True):
    """The reference's path-A attention in fp32 on the operands, as (B,S,H,D)."""
    dt = ops.q.dtype
    s = ops.s
    q = ops.q[:, :, :s].float()
    k = ops.k[:, :, :s].float()
    v = ops.v_t[..., :s].float().transpose(-1, -2).clone()
    if swap_keys is not None:
        i, j = swap_keys
        v[:, :, [i, j]] = v[:, :, [j, i]]
    main = q @ k.transpose(-1, -2)
    if ops.bias is None:
        p = torch.softmax(main * (sm * scale), dim=-1)
        o = (p @ v).to(dt)
    else:
        if round_main:
            main = main.to(dt).float()
        grp = ((torch.arange(s) // ops.q_group) + group_shift).clamp_max(ops.bias.shape[2] - 1)
        u = main * (sm * scale * LOG2E) + ops.bias[:, :, grp, :s]
        p = torch.softmax(u * math.log(2.0), dim=-1).to(dt).float()
        o = (p @ v).to(dt)
    return o.permute(0, 2, 1, 3).contiguous()


def test_fp32_evaluation_passes_no_qm():
    ops = _operands(1)
    sm = ops.d ** -0.5
    st = parity.sdpa_replay(ops, _fp32_attention(ops, sm), sm)
    assert st["excess"] <= 1.0 and st["frac_equal"] > 0.99, st


def test_fp32_evaluation_passes_qm_branch():
    ops = _operands(2, groups=4, q_group=64)
    sm = ops.d ** -0.5
    st = parity.sdpa_replay(ops, _fp32_attention(ops, sm), sm)
    assert st["excess"] <= 1.0 and st["frac_equal"] > 0.99, st


def test_fp16_evaluation_passes():
    ops = _operands(3, groups=4, q_group=48, dt=torch.float16)
    sm = ops.d ** -0.5
    st = parity.sdpa_replay(ops, _fp32_attention(ops, sm), sm)
    assert st["excess"] <= 1.0, st


def test_planted_wrong_scale_fails():
    ops = _operands(4)
    sm = ops.d ** -0.5
    assert parity.sdpa_replay(ops, _fp32_attention(ops, sm, scale=1.01), sm)["excess"] > 1.0


def test_planted_swapped_v_rows_fail():
    ops = _operands(5)
    sm = ops.d ** -0.5
    assert parity.sdpa_replay(ops, _fp32_attention(ops, sm, swap_keys=(3, 150)), sm)["excess"] > 1.0


def test_planted_wrong_group_fails():
    ops = _operands(6, groups=4, q_group=64)
    sm = ops.d ** -0.5
    assert parity.sdpa_replay(ops, _fp32_attention(ops, sm, group_shift=1), sm)["excess"] > 1.0


def test_planted_unrounded_main_score_fails():
    ops = _operands(7, groups=4, q_group=64)
    sm = ops.d ** -0.5
    assert parity.sdpa_replay(ops, _fp32_attention(ops, sm, round_main=False), sm)["excess"] > 1.0


def test_planted_three_ulp_error_fails():
    ops = _operands(8)
    sm = ops.d ** -0.5
    out = _fp32_attention(ops, sm)
    x = out[0, 17, 1, 5].float()
    out[0, 17, 1, 5] = (x + 3 * parity.ulp_dt(x, out.dtype).float()).to(out.dtype)
    assert parity.sdpa_replay(ops, out, sm)["excess"] > 1.0


def test_row_subsets_and_per_head_rows_agree():
    ops = _operands(9, groups=4, q_group=64)
    sm = ops.d ** -0.5
    out = _fp32_attention(ops, sm)
    rows = torch.tensor([0, 5, 63, 64, 199])
    a = parity.sdpa_replay(ops, out, sm, rows=rows)
    b = parity.sdpa_replay(ops, out, sm, rows=rows.expand(ops.h, -1))
    assert a == b and a["excess"] <= 1.0
