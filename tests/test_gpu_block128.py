"""block_n = 128 (attention_triton.py BLOCK_N = 128): the row-max update, P
scale and BLASST decision cover two 64-key MFMA tiles.  Checked as the 64-key
kernel is: the output against the reference algorithm replayed on the kernel's
own scores with block_n = 128 (rounding-edge flip
allowance), the BLASST statistics, per-row skip counts and per-wave skip
counters exactly, the reference bounded by its own bf16-vs-fp32-dequant gap
and the MFMA score-error gap (parity.reference_bound, BLASST included), and
-- dense -- cosine >= 0.9999 against the reference with its own scores.
Also the rowmax_init argument (attention_triton.py:127-130) at both block
sizes.
"""

import zlib

import pytest
import torch

import parity
from oracle import pipeline as opipe

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    from low_bit_fake_quant import QuantConfig
    base = dict(p_requant=True, p_requant_block_m=128, p_requant_block_n=128)
    base.update(kw)
    return QuantConfig(**base)


def _inputs(h=2, n=1024, d=128, seed=0, q_clusters=0, v_bias=False, field=None):
    from low_bit_fake_quant.wan import Workload, make_inputs
    w = Workload("t", h, n, d, None, q_clusters=q_clusters, v_bias=v_bias, field_grid=field)
    return make_inputs(w, seed=seed)


def _check(out, q, k, v, cfg, label, gpu, dense=True):
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    u = parity.kernel_scores(ops, cfg, sm)
    _, _, rep, dbg = parity.check_against_replay(out, q, k, v, cfg, ops, u, label)
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    ref32 = opipe.fake_quant_attention(q, k, v, cfg, qk_dequant_dtype=torch.float32)
    st = parity.reference_bound(out, ref, ref32, rep, label, allowance=dbg["flip_allowance_nhd"])
    if dense and st["ref_self_cos"] >= parity.COS_MIN:
        assert st["cos_ref"] >= parity.COS_MIN, f"{label}: vs reference cos={st['cos_ref']:.7f}"


CASES = {
    "elementwise_online_konly": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="k_only", q_kmeans_k=None,
                                     p_quant="elementwise"),
    "dynamic_qmk_full_kmeans": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full",
                                    q_smooth_block_size=256, q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k"),
    "mx_everything": dict(qk_quant="mxfp8", qk_hadamard=True, v_quant="mxfp8", v_mxfp8_block_size=64,
                          v_smooth_mode="per_block", v_smooth_block_size=128, smoothing="full", q_kmeans_k=16,
                          p_quant="mx", p_mx_block_n=128),
    "fp8blockV_dynamic_online": dict(qk_quant="fp8_block", fp8_block_size=128, v_quant="fp8_block",
                                     v_fp8_block_size=128, smoothing="off", q_kmeans_k=None, p_quant="dynamic"),
    "channelV_elementwise_vsmooth": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full",
                                         q_smooth_block_size=128, q_kmeans_k=None, p_quant="elementwise",
                                         v_smooth_mode="per_block", v_smooth_block_size=256),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_block128_matches_oracle(gpu, name):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES[name])
    q, k, v = _inputs(seed=zlib.crc32(name.encode()) % 1000, q_clusters=8, v_bias=True)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    _check(out, q, k, v, cfg, name, gpu)


@pytest.mark.parametrize("n", [960, 1000])
def test_block128_ragged(gpu, n):
    """S = 960: the last block's second tile is past S (all keys masked);
    S = 1000: it holds 40 valid keys."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="mxfp8", smoothing="k_only", q_kmeans_k=None, p_quant="dynamic")
    q, k, v = _inputs(n=n, seed=n)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    _check(out, q, k, v, cfg, f"ragged{n}", gpu)


FILLS = ["zero", "max_a0.25", "mean_a1.5", "logn", "sample8_a1.25", "thr_a0.25", "uta16_a1.5", "uta4", "uta1",
         "uta32", "uta64_a1.5", "uta128"]


@pytest.mark.parametrize("fill", FILLS)
def test_block128_blasst_fill_matches_oracle(gpu, fill):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
               q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05, blasst_fill=fill)
    q, k, v = _inputs(n=1024, seed=15, field=(4, 16, 16))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    _check(out, q, k, v, cfg, fill, gpu, dense=False)


@pytest.mark.parametrize("fill", ["mean_a1.5", "sample8_a1.25", "uta16_a1.5", "uta128"])
def test_block128_blasst_ragged(gpu, fill):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="mxfp8", smoothing="k_only", q_kmeans_k=None, p_quant="elementwise",
               blasst_lambda=0.05, blasst_fill=fill)
    q, k, v = _inputs(n=1000, seed=16, field=(4, 10, 25))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    _check(out, q, k, v, cfg, fill + "/ragged", gpu, dense=False)


@pytest.mark.parametrize("p_quant", ["elementwise", "mx", "dynamic"])
def test_block128_blasst_decisions_exact(gpu, p_quant):
    """Stats, per-row skip counts and per-wave counters equal the replay's."""
    from low_bit_fake_quant.attention_kernel import launch_attention
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="off", q_kmeans_k=None, p_quant=p_quant,
               p_mx_block_n=128, blasst_lambda=0.1, blasst_fill="mean_a1.5")
    q, k, v = _inputs(n=1024, seed=17, field=(4, 16, 16))
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    out, stats, rsk, wt = launch_attention(ops, cfg, sm, torch.bfloat16, return_blasst_stats=True,
                                           return_row_skips=True, return_wave_tiles=True)
    u = parity.kernel_scores(ops, cfg, sm)
    rep, rstats, dbg = parity.replay(q, k, v, cfg, ops, u, return_blasst_stats=True)
    stats = stats.cpu()
    assert stats[..., 0].sum() / stats[..., 1].sum() > 0.05, "test input should make BLASST skip"
    assert torch.equal(stats, rstats)
    assert torch.equal(rsk.cpu(), dbg["row_skips"].reshape(ops.b * ops.h, ops.s))
    sk = torch.stack(dbg["skip"], -1).reshape(ops.b * ops.h, ops.s, -1)  # 128-key blocks
    nw = wt.shape[1]
    skw = torch.zeros(ops.b * ops.h, nw * 32, sk.shape[-1], dtype=torch.bool)
    skw[:, :ops.s] = sk
    skw = skw.view(ops.b * ops.h, nw, 32, -1)
    assert torch.equal(wt[..., 0].cpu(), skw.all(2).sum(-1).int())
    assert torch.equal(wt[..., 1].cpu(), skw.any(2).sum(-1).int())
    parity.strict_check(out.cpu(), rep, f"decisions-{p_quant}", allowance=dbg["flip_allowance_nhd"])


@pytest.mark.parametrize("block_n", [64, 128])
@pytest.mark.parametrize("blasst", [False, True])
def test_rowmax_init_matches_oracle(gpu, block_n, blasst):
    """rowmax_init (attention_triton.py:127-130): the diagonal score of each
    row (the block studies' diagonal_rowmax_init), as the kernel forms it,
    starts the online max; the oracle replays with the same values."""
    from low_bit_fake_quant.attention_kernel import launch_attention
    kw = dict(blasst_lambda=0.05, blasst_fill="mean_a1.5") if blasst else {}
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=128, v_quant="fp8_block", v_fp8_block_size=128,
               smoothing="off", q_kmeans_k=None, p_quant="elementwise", p_requant_block_m=block_n,
               p_requant_block_n=block_n, **kw)
    q, k, v = _inputs(n=1024, seed=18 + block_n, field=(4, 16, 16))
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    u = parity.kernel_scores(ops, cfg, sm)                      # (B,H,S,S) log2 units
    init = torch.diagonal(u, dim1=-2, dim2=-1).contiguous()     # (B,H,S)
    out = launch_attention(ops, cfg, sm, torch.bfloat16,
                           rowmax_init=init.reshape(ops.b * ops.h, ops.s).to(gpu))
    rep, dbg = parity.replay(q, k, v, cfg, ops, u, rowmax_init=init / parity.LOG2E)
    parity.strict_check(out.cpu(), rep, f"init{block_n}-{blasst}", allowance=dbg["flip_allowance_nhd"])
    # the initial value matters: without it the result differs (elementwise P)
    plain = launch_attention(ops, cfg, sm, torch.bfloat16)
    assert not torch.equal(plain, out)
