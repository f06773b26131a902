"""Diagnostic probes on the GPU against the CPU oracle (``oracle/probe.py``).

* ``p_requant_rows`` (reference ``p_requant.py``): P codes equal the oracle's
  except where the GPU and CPU ``exp2`` (each within an ulp or so) round to
  neighbouring E4M3 codes -- at most 0.2% of codes, one step apart; row sums
  within 2e-6 relative (summation order); lse within 2e-6 absolute.
* rowmax counters (reference ``bench/count_rowmax_updates_triton.py``): on
  the kernel's own scores (FP8 codes, log2 units, restated by the oracle)
  the six counters are equal; against the reference's bf16-dequantised
  scores they agree within 2% (+2), the rows where the two score roundings
  fall on different sides of a threshold.
"""

import json

import pytest
import torch

from conftest import cpu_randn
from oracle import probe as oprobe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("off", [8, 10])
def test_p_requant_rows_matches_oracle(gpu, dtype, off):
    from low_bit_fake_quant.p_requant import p_requant_rows
    x = (cpu_randn(3, 37, 300, seed=5, dtype=torch.float32) * 4.0).to(dtype)
    # a strided view: every other column of a wider matrix
    wide = torch.zeros(3, 37, 600, dtype=dtype)
    wide[..., ::2] = x
    xs = wide.to(gpu)[..., ::2]
    sm = 128 ** -0.5
    p, rs, lse = p_requant_rows(xs, sm_scale=sm, p_max_offset=off)
    assert p.dtype == torch.float8_e4m3fn and p.shape == x.shape
    codes, rs_o, lse_o = oprobe.p_requant_rows(x.float(), sm_scale=sm, p_max_offset=off)
    got = p.cpu().view(torch.uint8)
    diff = got.int() != codes.int()
    assert diff.float().mean().item() <= 2e-3
    assert ((got.int() - codes.int()).abs()[diff] <= 1).all()
    assert torch.allclose(rs.cpu(), rs_o, rtol=2e-6, atol=0)
    assert torch.allclose(lse.cpu(), lse_o, rtol=0, atol=2e-6)


def test_p_requant_rows_errors(gpu):
    from low_bit_fake_quant.p_requant import p_requant_rows
    with pytest.raises(ValueError, match="3-D CUDA"):
        p_requant_rows(torch.zeros(4, 8, device=gpu), sm_scale=1.0)
    with pytest.raises(ValueError, match="3-D CUDA"):
        p_requant_rows(torch.zeros(1, 4, 8), sm_scale=1.0)
    with pytest.raises(ValueError, match="block_n=4 must be >= N=8"):
        p_requant_rows(torch.zeros(1, 4, 8, device=gpu), sm_scale=1.0, block_n=4)


def _counter_case(gpu, seed=0, s=1024, h=2, q_group=256):
    from low_bit_fake_quant.attention import _lazy_preprocess, quantize_operands
    from low_bit_fake_quant.rowmax_counters import counter_config
    cfg = counter_config(q_kmeans_k=8, q_smooth_block=q_group)
    q = cpu_randn(1, s, h, 128, seed=seed + 1)
    k = (cpu_randn(1, s, h, 128, seed=seed + 2).float() * 2.0
         + cpu_randn(1, 1, h, 128, seed=seed + 4).float() * 3.0).to(torch.bfloat16)
    v = cpu_randn(1, s, h, 128, seed=seed + 3)
    sm = 128 ** -0.5
    ops = quantize_operands(_lazy_preprocess(q.to(gpu), k.to(gpu), v.to(gpu), cfg), cfg, sm)
    return cfg, q, k, v, ops, sm


PAIRS = [(8.0, 8.0), (16.0, 32.0), (2.0, 4.0)]


@pytest.mark.parametrize("s,q_group", [(1024, 256), (320, 64)])
def test_rowmax_counts_match_oracle_on_kernel_scores(gpu, s, q_group):
    """Counters equal the oracle's on the kernel's own scores.  S = 320 leaves
    the last 128-row workgroup with two waves past the rows, which still stage
    their share of every K tile and meet every barrier but count nothing."""
    from low_bit_fake_quant.rowmax_counters import count_rowmax_updates
    cfg, q, k, v, ops, sm = _counter_case(gpu, s=s, q_group=q_group)
    u2, est2 = oprobe.kernel_scores_log2(ops.q_codes.cpu(), ops.q_scale.cpu(), ops.k_codes.cpu(), ops.k_scale.cpu(),
                                         ops.bias.cpu(), ops.rowmax.cpu(), s=ops.s, qk_block=cfg.fp8_block_size,
                                         q_group=cfg.q_smooth_block_size, sm_scale=sm)
    for up, down in PAIRS:
        for est in (False, True):
            got = count_rowmax_updates(ops, cfg, sm_scale=sm, up_threshold=up, down_threshold=down,
                                       use_estimate=est)
            ref = oprobe.rowmax_counts(u2, est2, up=up, down=down, use_estimate=est, units="log2")
            assert got == ref, (up, down, est, got, ref)
            # the online rule updates at least once per row (its first tile)
            assert est or got["rows_with_update"] == ops.b * ops.h * ops.s


def test_rowmax_counts_close_to_reference_scores(gpu):
    from low_bit_fake_quant.rowmax_counters import count_rowmax_updates
    cfg, q, k, v, ops, sm = _counter_case(gpu, seed=10)
    s_nat, est_nat = oprobe.reference_scores(q, k, v, cfg, sm_scale=sm)
    for up, down in PAIRS:
        for est in (False, True):
            got = count_rowmax_updates(ops, cfg, sm_scale=sm, up_threshold=up, down_threshold=down,
                                       use_estimate=est)
            ref = oprobe.rowmax_counts(s_nat, est_nat, up=up, down=down, use_estimate=est, units="natural")
            for name in oprobe.COUNTER_NAMES:
                assert abs(got[name] - ref[name]) <= 2 + 0.02 * ref[name], (up, down, est, name, got, ref)


def test_rowmax_counter_cli(gpu, tmp_path):
    from low_bit_fake_quant import rowmax_counters
    q = cpu_randn(1, 1000, 2, 128, seed=31)
    k = cpu_randn(1, 1000, 2, 128, seed=32)
    v = cpu_randn(1, 1000, 2, 128, seed=33)
    dump = tmp_path / "call_000.pt"
    torch.save({"query": q, "key": k, "value": v, "record": {"kind": "self-fq"}}, dump)
    out = tmp_path / "counts.json"
    rep = rowmax_counters.main(["--workload", str(dump), "--output", str(out), "--q-kmeans-k", "8",
                                "--up-thresholds", "16", "--down-thresholds", "32"])
    assert rep["shape"] == [1, 1024, 2, 128] and rep["pad"] == 24
    r = json.loads(out.read_text())["results"]["up16.0_down32.0"]
    rows = 1024 * 2
    for name in ("fa4_online", "estimated"):
        assert r[name]["rows_with_update"] <= rows
        assert r[name]["updates_per_row_avg"] == r[name]["updates"] / rows
    # the online rule always updates on the first tile of every row
    assert r["fa4_online"]["rows_with_update"] == rows
