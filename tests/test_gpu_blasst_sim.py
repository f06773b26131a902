"""BLASST tile-skip simulator on the GPU (``low_bit_fake_quant.blasst_skip``)
against the CPU oracle (``oracle/blasst_sim.py``), plus the reference's own
GPU cases (``tests/test_blasst_skip.py``) restated.

Tolerance: outputs within cosine 0.99999 and max |diff| <= 2e-3 max|ref|
(fp32 sums in another order move a few P weights across a bf16 rounding
boundary); skip rates, forced tiles and the Q/K/V quant counts equal; P
statistics and dropped-mass quantiles within 1e-4 absolute / 1e-3 relative
(exp rounding moves a handful of P values across an E4M3 boundary).
"""

import math

import pytest
import torch

from conftest import cpu_randn
from oracle import blasst_sim as osim

pytestmark = pytest.mark.gpu


def _close(a, b, cos_min=0.99999, rel_max=2e-3):
    a, b = a.double().flatten(), b.double().flatten()
    cos = float(a @ b / (a.norm() * b.norm()))
    m = float((a - b).abs().max())
    assert cos >= cos_min and m <= rel_max * float(b.abs().max()), (cos, m)


def _qkv(s, h, d, seed, skippable=False):
    q = cpu_randn(1, s, h, d, seed=seed)
    k = cpu_randn(1, s, h, d, seed=seed + 1)
    v = cpu_randn(1, s, h, d, seed=seed + 2)
    if skippable:
        k = k.float()
        k[:, :128] *= 8.0
        k[:, 128:] *= 0.02
        k = k.to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("d,mm,s", [(64, torch.bfloat16, 512), (128, torch.bfloat16, 512), (64, torch.float32, 512),
                                    (128, torch.float32, 128), (128, torch.bfloat16, 384), (64, torch.bfloat16, 384)])
def test_simulator_matches_oracle(gpu, d, mm, s):
    """S = 128 is one query tile and one key block (the scan's slice prefetch
    wraps onto its last slice at once); S = 384 is three of each."""
    from low_bit_fake_quant import blasst_skip as bs
    q, k, v = _qkv(s, 2, d, seed=40 + d + s, skippable=True)
    ths = [0.0, 0.05, 0.9, 2.0]
    res = bs.simulate_workload(q.to(gpu), k.to(gpu), v.to(gpu), skip_thresholds=ths, matmul_dtype=mm)
    ref = osim.simulate(q, k, v, skip_thresholds=ths, mm_dtype=mm)
    for lv in ("bf16_ref", "fp8_qkv", "fp8_static_p"):
        _close(res.outputs[lv][0].cpu(), ref[lv])
    for th in ths:
        _close(res.skip_outputs[th][0].cpu(), ref["skip"][th])
        dg = res.skip_diagnostics[th]
        assert dg.skip_rate == ref["skip_rate"][th] and dg.force_keep_count == ref["force"][th]
        dm = ref["dropped"][th].flatten().sort().values
        n = dm.numel()
        assert abs(dg.dropped_mass_mean - float(dm.mean())) < 1e-4
        assert abs(dg.dropped_mass_max - float(dm[-1])) < 1e-4
        assert abs(dg.dropped_mass_median - float(dm[(n - 1) // 2])) < 1e-4
    # one key block (S = 128) is always kept by the empty-tile safeguard
    assert res.skip_diagnostics[0.0].skip_rate == 0.0 and (s == 128 or res.skip_diagnostics[0.9].skip_rate > 0.0)
    for name in ("q", "k", "v"):
        st, so = res.quant_stats[name], ref["stats"][name]
        assert st.saturation_rate == so["saturation_rate"] and st.underflow_zero_rate == so["underflow_zero_rate"]
        assert abs(st.roundtrip_rmse - so["roundtrip_rmse"]) <= 1e-6 * so["roundtrip_rmse"] + 1e-12
    sp, op = res.quant_stats["p"], ref["stats"]["p"]
    assert abs(sp.underflow_zero_rate - op["underflow_zero_rate"]) < 1e-4
    assert abs(sp.roundtrip_rmse - op["roundtrip_rmse"]) <= 1e-3 * op["roundtrip_rmse"]


def test_reference_rung_matches_dense_fp32(gpu):
    from low_bit_fake_quant import blasst_skip as bs
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 512, 3, 64, dtype=torch.bfloat16) for _ in range(3))
    res = bs.simulate_workload(q.to(gpu), k.to(gpu), v.to(gpu), skip_thresholds=[], levels=[bs.LEVEL_REFERENCE],
                               matmul_dtype=torch.float32)
    qf, kf, vf = (t[0].double().permute(1, 0, 2) for t in (q, k, v))
    ref = (torch.softmax(qf @ kf.transpose(1, 2) / 8.0, -1) @ vf).permute(1, 0, 2)
    pred = res.outputs[bs.LEVEL_REFERENCE][0].cpu().double()
    cos = float((pred.flatten() @ ref.flatten()) / (pred.norm() * ref.norm()))
    assert cos >= 0.9999 and float((pred - ref).norm() / ref.norm()) <= 1e-3
    # a 1/d softmax scale (instead of 1/sqrt(d)) must not pass the same check
    res2 = bs.simulate_workload((q.float() * 8.0 / 64.0).to(torch.bfloat16).to(gpu), k.to(gpu), v.to(gpu),
                                skip_thresholds=[], levels=[bs.LEVEL_REFERENCE], matmul_dtype=torch.float32)
    p2 = res2.outputs[bs.LEVEL_REFERENCE][0].cpu().double()
    assert float((p2.flatten() @ ref.flatten()) / (p2.norm() * ref.norm())) < 0.999


def test_skip_zero_equals_no_skip_bitwise(gpu):
    from low_bit_fake_quant import blasst_skip as bs
    q, k, v = _qkv(512, 2, 64, seed=2)
    res = bs.simulate_workload(q.to(gpu), k.to(gpu), v.to(gpu), skip_thresholds=[0.0],
                               levels=[bs.LEVEL_FP8_STATIC_P, bs.LEVEL_FP8_SKIP])
    assert torch.equal(res.outputs[bs.LEVEL_FP8_STATIC_P], res.skip_outputs[0.0])
    assert res.skip_diagnostics[0.0].skip_rate == 0.0


def test_skip_rate_monotone_and_safeguard(gpu):
    from low_bit_fake_quant import blasst_skip as bs
    q, k, v = _qkv(1024, 2, 64, seed=3, skippable=True)
    res = bs.simulate_workload(q.to(gpu), k.to(gpu), v.to(gpu), skip_thresholds=[0.0, 0.1, 0.9, 1.0],
                               levels=[bs.LEVEL_FP8_SKIP])
    r = [res.skip_diagnostics[t].skip_rate for t in (0.0, 0.1, 0.9)]
    assert r[0] == 0.0 and r[0] <= r[1] <= r[2] and 0.0 < r[2] <= 1.0
    assert torch.isfinite(res.skip_outputs[1.0]).all()


def test_reorder_lambda0_equivalence(gpu):
    from low_bit_fake_quant import blasst_skip as bs
    t, h, w = 8, 8, 16
    s = t * h * w
    q, k, v = (x.to(gpu) for x in _qkv(s, 2, 64, seed=6))
    native = bs.simulate_workload(q, k, v, skip_thresholds=[], levels=[bs.LEVEL_REFERENCE])
    perm = bs.space_time_reorder_index(t, h, w, device=q.device)
    inv = bs.invert_permutation(perm)
    re = bs.simulate_workload(*(bs.apply_token_permutation(x, perm) for x in (q, k, v)), skip_thresholds=[],
                              levels=[bs.LEVEL_REFERENCE])
    o_nat = native.outputs[bs.LEVEL_REFERENCE]
    o_back = bs.apply_token_permutation(re.outputs[bs.LEVEL_REFERENCE], inv)
    _close(o_back.cpu(), o_nat.cpu(), cos_min=0.99999, rel_max=1e-2)
    a, b = re.outputs[bs.LEVEL_REFERENCE].flatten().double(), o_nat.flatten().double()
    assert float(a @ b / (a.norm() * b.norm())) < 0.9999


def test_per_head_quant_and_guards(gpu):
    from low_bit_fake_quant import blasst_skip as bs
    x = (cpu_randn(256, 4, 64, seed=5, dtype=torch.float32) * 7.0).to(torch.bfloat16)
    deq, scale, st = bs.fake_quant_per_head(x.to(gpu))
    assert scale.shape == (1, 4, 1) and deq.shape == x.shape and st.saturation_rate < 1e-4
    d_o, s_o, st_o = osim.head_quant(x)
    assert torch.equal(deq.cpu(), d_o) and torch.equal(scale.view(-1).cpu(), s_o)
    q = torch.randn(1, 200, 2, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        bs.simulate_workload(q, q, q, skip_thresholds=[], levels=[bs.LEVEL_REFERENCE])
    z = torch.zeros(1, bs.MATH_BACKEND_SEQLEN_LIMIT, 1, 8, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(bs.FullMatrixAllocationError):
        bs.sdpa_ground_truth(z, z, z, force_math_backend=True)
    qs = torch.randn(1, 256, 1, 8, dtype=torch.bfloat16, device=gpu)
    assert bs.sdpa_ground_truth(qs, qs, qs, force_math_backend=True).shape == qs.shape
