"""P-requant FP8-MFMA attention vs the CPU oracle of the reference path.

Tolerances (north star: cosine >= 0.9999, max |diff| <= 1e-2), see
``tests/parity.py`` for the full argument:

* the kernel's scores equal the exact scores of its FP8 codes within the
  measured accumulation error of the gfx950 FP8 MFMA (2^-10 * max|a| * max|b|
  per MFMA, ~3x the largest error observed);
* the kernel's output equals the reference algorithm replayed on the kernel's
  own scores (oracle, ``attention_triton.py:163-407``): cosine >= 0.9999 and
  every |diff| <= 1e-2, or one bf16 ulp of the value where that is larger
  (both sides round an fp32 value to bf16); BLASST per-row skip counts and
  statistics exactly;
* against the reference's own bf16-dequant scores, every configuration
  (BLASST included): element-wise within the larger of the reference's own
  bf16-vs-fp32 dequant gap and the MFMA score-error gap on the same rows plus
  the strict tolerance, and the angle to the reference within the larger of
  the two gaps' angles plus acos(0.9999) (``parity.reference_bound``); cosine
  >= 0.9999 against the reference for the dense configurations wherever the
  reference itself keeps 0.9999 against its exact-dequant variant; BLASST
  skip decisions equal outside rows within the score perturbation of the
  threshold.  The remaining element-wise gap is the reference's bf16
  rounding of the dequantised Q/K (attention.py:534-535) and the MFMA
  accumulation acting on the scores, which an FP8-MFMA kernel cannot
  reproduce.
Codes, scales and permutations are checked bit-exactly in the other GPU
tests.
"""

import dataclasses
import zlib

import pytest
import torch

import parity
from conftest import cosine, max_abs
from oracle import pipeline as opipe

pytestmark = pytest.mark.gpu

COS_MIN = parity.COS_MIN
MAXABS = parity.MAXABS


def check_parity(out, q, k, v, cfg, label="", dev=None):
    """Strict check against the replay; against the reference bounded by the
    reference's own bf16-vs-fp32-dequant gap (every configuration); cosine
    against the reference (dense)."""
    dev = dev or torch.device("cuda:0")
    ops, sm = parity.kernel_operands(q, k, v, cfg, dev)
    u = parity.kernel_scores(ops, cfg, sm)
    c_rep, m_rep, rep, dbg = parity.check_against_replay(out, q, k, v, cfg, ops, u, label)
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    ref32 = opipe.fake_quant_attention(q, k, v, cfg, qk_dequant_dtype=torch.float32)
    st = parity.reference_bound(out, ref, ref32, rep, label, allowance=dbg["flip_allowance_nhd"])
    if cfg.blasst_lambda is None and st["ref_self_cos"] >= COS_MIN:
        assert st["cos_ref"] >= COS_MIN, f"{label}: vs reference cos={st['cos_ref']:.7f}"
    return c_rep, m_rep, st["cos_ref"]


def _cfg(**kw):
    from low_bit_fake_quant import QuantConfig
    base = dict(p_requant=True, p_requant_block_m=64, p_requant_block_n=64)
    base.update(kw)
    return QuantConfig(**base)


def _inputs(h=2, n=1024, d=128, seed=0, q_clusters=0, v_bias=False, dtype=torch.bfloat16, field=None):
    from low_bit_fake_quant.wan import Workload, make_inputs
    w = Workload("t", h, n, d, None, q_clusters=q_clusters, v_bias=v_bias, field_grid=field)
    return make_inputs(w, seed=seed, dtype=dtype)


CASES = {
    "c1_elementwise_online_konly": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel",
                                        smoothing="k_only", q_kmeans_k=None, p_quant="elementwise"),
    "c2_dynamic_qmk_full_kmeans": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel",
                                       smoothing="full", q_smooth_block_size=256, q_kmeans_k=32,
                                       p_quant="dynamic", rowmax_mode="qm_k"),
    "c3_mxfp8_everything": dict(qk_quant="mxfp8", qk_hadamard=True, v_quant="mxfp8", v_mxfp8_block_size=64,
                                v_kmeans_k=64, v_smooth_mode="per_block", v_smooth_block_size=64,
                                smoothing="full", q_kmeans_k=32, p_quant="mx"),
    "dynamic_online": dict(qk_quant="fp8_block", fp8_block_size=128, v_quant="fp8_channel", smoothing="full",
                           q_smooth_block_size=128, q_kmeans_k=None, p_quant="dynamic"),
    "elementwise_qmk_fixed": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full",
                                  q_smooth_block_size=256, q_kmeans_k=16, p_quant="elementwise",
                                  rowmax_mode="qm_k"),
    "mx_qmk_fixed_fp8blockV": dict(qk_quant="mxfp8", v_quant="fp8_block", v_fp8_block_size=128,
                                   smoothing="full", q_smooth_block_size=128, q_kmeans_k=None, p_quant="mx",
                                   p_mx_block_n=64, rowmax_mode="qm_k"),
    "fp8blockV_elementwise_vsmooth": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_block",
                                          v_fp8_block_size=64, smoothing="off", q_kmeans_k=None,
                                          v_smooth_mode="per_block", v_smooth_block_size=128),
    "channelV_dynamic_vsmooth": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel",
                                     smoothing="full", q_smooth_block_size=256, q_kmeans_k=None,
                                     p_quant="dynamic", v_smooth_mode="per_block", v_smooth_block_size=64),
    "blasst_mean_vsmooth": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_block", v_fp8_block_size=64,
                                smoothing="off", q_kmeans_k=None, p_quant="elementwise", v_smooth_mode="per_block",
                                v_smooth_block_size=64, blasst_lambda=0.05, blasst_fill="mean_a1.5"),
    "default_config": dict(),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_attention_matches_oracle(gpu, name):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES[name])
    q, k, v = _inputs(seed=zlib.crc32(name.encode()) % 1000, q_clusters=8, v_bias=True)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    check_parity(out, q, k, v, cfg, name)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attention_dtypes_and_head_dims(gpu, d, dtype):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES["c2_dynamic_qmk_full_kmeans"])
    q, k, v = _inputs(n=512, d=d, seed=3, q_clusters=4, dtype=dtype)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    assert out.dtype == dtype
    check_parity(out, q, k, v, cfg, f"{dtype}-{d}")


def test_ragged_sequence_length(gpu):
    """S not a multiple of the 128-query workgroup (masked keys in the last tile)."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="off", q_kmeans_k=None, p_quant="elementwise")
    q, k, v = _inputs(n=1000, d=128, seed=4)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    check_parity(out, q, k, v, cfg, "ragged")


@pytest.mark.parametrize("fill", ["zero", "max_a0.25", "mean_a1.5", "logn", "sample8_a1.25", "thr_a0.25",
                                  "uta16_a1.5", "uta4", "uta2_a1.5", "uta", "uta1", "uta8", "uta64_a1.5"])
def test_blasst_fill_matches_oracle(gpu, fill):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
               q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05, blasst_fill=fill)
    q, k, v = _inputs(n=1024, seed=5, field=(4, 16, 16))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    check_parity(out, q, k, v, cfg, fill)


@pytest.mark.parametrize("fill", ["mean_a1.5", "logn", "sample8_a1.25", "uta16_a1.5", "uta1"])
def test_blasst_fill_ragged_matches_oracle(gpu, fill):
    # S = 1000: the last 64-key tile holds 40 valid keys (masked fill statistics)
    from low_bit_fake_quant import fake_quant_attention
    # (fp8_block and Q smoothing need S divisible by their blocks: MX Q/K, K-only
    # smoothing, online row max)
    cfg = _cfg(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="k_only", q_kmeans_k=None,
               p_quant="dynamic", rowmax_mode="online", blasst_lambda=0.05, blasst_fill=fill)
    q, k, v = _inputs(n=1000, seed=6, field=(4, 10, 25))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    check_parity(out, q, k, v, cfg, fill + "/ragged")


@pytest.mark.parametrize("p_quant", ["elementwise", "mx", "dynamic"])
def test_blasst_stats_match_oracle(gpu, p_quant):
    """Stats (attention_triton.py:404-407) equal the replay's exactly."""
    from low_bit_fake_quant.attention_kernel import launch_attention
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="off", q_kmeans_k=None, p_quant=p_quant,
               p_mx_block_n=64, blasst_lambda=0.1, blasst_fill="mean_a1.5")
    q, k, v = _inputs(n=1024, seed=6, field=(4, 16, 16))
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    out, stats = launch_attention(ops, cfg, sm, torch.bfloat16, return_blasst_stats=True)
    u = parity.kernel_scores(ops, cfg, sm)
    rep, rstats, dbg = parity.replay(q, k, v, cfg, ops, u, return_blasst_stats=True)
    stats = stats.cpu()
    assert stats[..., 0].sum() / stats[..., 1].sum() > 0.05, "test input should make BLASST skip"
    assert torch.equal(stats, rstats)
    parity.strict_check(out.cpu(), rep, f"stats-{p_quant}", allowance=dbg["flip_allowance_nhd"])


SKIP_CASES = {
    "dyn_qmk_mean": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                         q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k", blasst_fill="mean_a1.5"),
    "dyn_qmk_uta16": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                          q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k", blasst_fill="uta16_a1.5"),
    "elementwise_online_zero": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="k_only", q_kmeans_k=None,
                                    p_quant="elementwise", blasst_fill="zero"),
    "mx_qk_mx_p_logn": dict(qk_quant="mxfp8", v_quant="mxfp8", v_mxfp8_block_size=64, smoothing="k_only",
                            q_kmeans_k=None, p_quant="mx", blasst_fill="logn"),
    "uta64_vsmooth": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_block", v_fp8_block_size=64,
                          smoothing="off", q_kmeans_k=None, p_quant="dynamic", v_smooth_mode="per_block",
                          v_smooth_block_size=64, blasst_fill="uta64_a1.5"),
}


@pytest.mark.parametrize("name", sorted(SKIP_CASES))
def test_blasst_row_skips_bit_exact(gpu, name):
    """Per-row skip decisions (attention_triton.py:165-175): the kernel's
    per-row skipped-block counts equal the replay's exactly, and the
    reference's in every row whose predicate margin stays farther from the
    threshold than the score perturbation; the rows within it are counted."""
    from low_bit_fake_quant.attention_kernel import launch_attention
    cfg = _cfg(blasst_lambda=0.05, **SKIP_CASES[name])
    q, k, v = _inputs(n=1024, seed=zlib.crc32(name.encode()) % 1000, field=(4, 16, 16))
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    out, rsk, wt = launch_attention(ops, cfg, sm, torch.bfloat16, return_row_skips=True, return_wave_tiles=True)
    u = parity.kernel_scores(ops, cfg, sm)
    rep, dbg_rep = parity.replay(q, k, v, cfg, ops, u)
    order = dbg_rep["order"]
    rs_rep = parity.unpermute_rows(dbg_rep["row_skips"].reshape(ops.b * ops.h, ops.s), order)
    assert torch.equal(rsk.cpu(), rs_rep)
    assert rs_rep.sum() > 0, "test input should make BLASST skip"
    # per wave of 32 kernel rows: tiles that all / some of its rows skipped
    sk = torch.stack(dbg_rep["skip"], -1).reshape(ops.b * ops.h, ops.s, -1)
    nw = wt.shape[1]
    skw = torch.zeros(ops.b * ops.h, nw * 32, sk.shape[-1], dtype=torch.bool)
    skw[:, :ops.s] = sk
    skw = skw.view(ops.b * ops.h, nw, 32, -1)
    assert torch.equal(wt[..., 0].cpu(), skw.all(2).sum(-1).int())
    assert torch.equal(wt[..., 1].cpu(), skw.any(2).sum(-1).int())
    print(f"{name}: wave tiles all-skip {int(wt[..., 0].sum())}, some-skip {int(wt[..., 1].sum())}, "
          f"of {nw * ops.b * ops.h * sk.shape[-1]}")
    parity.strict_check(out.cpu(), rep, name, allowance=dbg_rep["flip_allowance_nhd"])
    ref, dbg_ref = opipe.fake_quant_attention(q, k, v, cfg, return_debug=True)
    compared, near, disagree = parity.skip_agreement(rsk, dbg_ref, u, order)
    print(f"{name}: rows compared {compared}, near the threshold {near}, disagreeing {disagree}")
    assert disagree == 0 and compared >= 0.5 * rsk.numel()


def test_mx_p_ignores_p_max_offset_bitwise(gpu):
    from low_bit_fake_quant import fake_quant_attention
    base = dict(qk_quant="mxfp8", v_quant="mxfp8", smoothing="off", q_kmeans_k=None, v_smooth_mode="off",
                v_mxfp8_block_size=64, p_quant="mx")
    q, k, v = (t.to(gpu) for t in _inputs(n=256, d=64, seed=11))
    o0 = fake_quant_attention(q, k, v, _cfg(**base, p_max_offset=0))
    o8 = fake_quant_attention(q, k, v, _cfg(**base, p_max_offset=8))
    assert (o0.float() - o8.float()).abs().max().item() == 0.0


def test_preprocess_cache_equivalent(gpu):
    from low_bit_fake_quant import fake_quant_attention, prepare_for_attention
    cfg = _cfg(**CASES["c3_mxfp8_everything"])
    q, k, v = (t.to(gpu) for t in _inputs(n=512, seed=12, q_clusters=4, v_bias=True))
    cache = prepare_for_attention(q, k, v, cfg)
    o1 = fake_quant_attention(q, k, v, cfg)
    o2 = fake_quant_attention(q, k, v, cfg, preprocess_cache=cache)
    assert torch.equal(o1, o2)
    with pytest.raises(ValueError, match="preprocess_cache does not match"):
        fake_quant_attention(q, k, v, dataclasses.replace(cfg, smoothing="off"), preprocess_cache=cache)


def test_sdpa_path_config0_matches_oracle(gpu):
    from low_bit_fake_quant import fake_quant_attention
    from low_bit_fake_quant.wan import make_inputs, workloads
    w = workloads()[0]
    q, k, v = make_inputs(w, seed=0)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), w.cfg).cpu()
    ref = opipe.fake_quant_attention(q, k, v, w.cfg)
    c, m = cosine(out, ref), max_abs(out, ref)
    assert c >= COS_MIN and m <= MAXABS, f"cos={c:.6f} maxabs={m:.3e}"


def test_sdpa_path_with_q_smoothing_and_kmeans(gpu):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(p_requant=False, smoothing="full", q_smooth_block_size=128, q_kmeans_k=8, qk_hadamard=True,
               v_smooth_mode="per_block", v_smooth_block_size=64)
    q, k, v = _inputs(n=512, d=64, seed=13, q_clusters=4)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    c, m = cosine(out, ref), max_abs(out, ref)
    assert c >= COS_MIN and m <= MAXABS, f"cos={c:.6f} maxabs={m:.3e}"


@pytest.mark.parametrize("name", ["c1_elementwise_online_konly", "c2_dynamic_qmk_full_kmeans", "c3_mxfp8_everything",
                                  "mx_qmk_fixed_fp8blockV", "fp8blockV_elementwise_vsmooth"])
def test_attention_is_deterministic(gpu, name):
    """Two calls on the same inputs give bitwise-identical outputs (the staged
    global->LDS copies are always complete before a tile's data is read)."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES[name])
    q, k, v = (t.to(gpu) for t in _inputs(n=4096, seed=31, q_clusters=8, v_bias=True))
    o1 = fake_quant_attention(q, k, v, cfg)
    o2 = fake_quant_attention(q, k, v, cfg)
    assert torch.equal(o1, o2)


def test_blasst_is_deterministic(gpu):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256, q_kmeans_k=16,
               p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05, blasst_fill="uta16_a1.5")
    q, k, v = (t.to(gpu) for t in _inputs(n=4096, seed=32, field=(4, 32, 32)))
    assert torch.equal(fake_quant_attention(q, k, v, cfg), fake_quant_attention(q, k, v, cfg))


def test_blasst_rows_with_every_block_skipped_match_oracle(gpu):
    """With the qm_k estimate above every tile max by more than |ln lambda|, a
    row can skip all its blocks; with the zero fill its mass is 0 and the
    reference's output row is 0/0.  The kernel's non-finite rows are exactly
    the oracle's and the finite rows keep parity."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256, q_kmeans_k=16,
               p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05, blasst_fill="zero")
    q, k, v = _inputs(n=1024, d=128, seed=24, q_clusters=4, v_bias=True, field=(4, 16, 16))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    bad_o, bad_r = ~torch.isfinite(out).all(-1), ~torch.isfinite(ref).all(-1)
    assert bad_r.any() and torch.equal(bad_o, bad_r)
    keep = ~bad_r
    assert cosine(out[keep], ref[keep]) >= COS_MIN


SCORE_CASES = ["c1_elementwise_online_konly", "c2_dynamic_qmk_full_kmeans", "c3_mxfp8_everything",
               "mx_qmk_fixed_fp8blockV", "dynamic_online"]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("name", SCORE_CASES)
def test_kernel_scores_match_exact_products(gpu, name, d):
    """The kernel's scores (its own MFMA sequence, lbfq_attention_scores) equal
    the exact float64 scores of its FP8 codes and scales plus its qm
    correction within the FP8 MFMA's accumulation bound; and they are not
    exact (the gfx950 FP8 MFMA does not accumulate in full fp32 precision)."""
    cfg = _cfg(**CASES[name])
    q, k, v = _inputs(n=512, d=d, seed=zlib.crc32(name.encode()) % 997, q_clusters=8, v_bias=True)
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    u = parity.kernel_scores(ops, cfg, sm).double()
    ue, bound = parity.exact_scores_and_bound(ops, cfg, sm)
    err = (u - ue).abs()
    ratio = (err / bound).max().item()
    print(f"{name}/d{d}: max |u - exact| = {err.max():.3e} (log2 units), max err/bound = {ratio:.3f}")
    assert ratio <= 1.0, f"{name}/d{d}: kernel score error exceeds the MFMA accumulation bound ({ratio:.2f}x)"


@pytest.mark.parametrize("name", ["c1_elementwise_online_konly", "c2_dynamic_qmk_full_kmeans", "dynamic_online"])
def test_reference_gap_comes_from_the_scores(gpu, name):
    """Where the kernel and the reference (bf16-dequant scores) differ.  The
    kernel equals the replay of the reference algorithm on its own scores
    (strict); the P codes that differ between the replay and the reference
    are single E4M3 steps whose pre-quantisation values straddle the
    rounding midpoint (scores on either side of a boundary); and the
    reference moves by more than 1e-2 under its own exact-arithmetic
    variant (fp32 dequant, attention.py:534-535), so 1e-2 element-wise is
    below the reference's own sensitivity on these inputs."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES[name])
    q, k, v = _inputs(seed=zlib.crc32(name.encode()) % 1000, q_clusters=8, v_bias=True)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
    u = parity.kernel_scores(ops, cfg, sm)
    _, _, rep, dbg_rep = parity.check_against_replay(out, q, k, v, cfg, ops, u, name)
    ref, dbg_ref = opipe.fake_quant_attention(q, k, v, cfg, return_debug=True)
    flips, one_step = parity.flipped_codes(dbg_ref, dbg_rep)
    assert one_step, f"{name}: a P code moved by more than one E4M3 step"
    r32 = opipe.fake_quant_attention(q, k, v, cfg, qk_dequant_dtype=torch.float32)
    ds = (u.double() / parity.LOG2E - dbg_ref["s"].double()).abs().max().item()
    print(f"{name}: max score gap {ds:.3e} (natural units), P codes flipped {flips.float().mean():.2e}, "
          f"max|kernel - ref| {max_abs(out, ref):.3e}, max|ref(fp32 dequant) - ref| {max_abs(r32, ref):.3e}, "
          f"cos(kernel, ref) {cosine(out, ref):.7f}")
    assert max_abs(r32, ref) > MAXABS


@pytest.mark.timeout(900)
@pytest.mark.parametrize("config", [1, 2, 3, 4])
def test_full_length_padded_wan_shapes(gpu, config):
    """BASELINE configs 1-4 at their real lengths (N = 32760, and 75600 for
    config 4, padded per the Wan hook: Q zero rows, K/V repeat the last row,
    bench/wan_attention_hook.py:249-294), 4 heads, 1024 random rows of the
    padded problem plus, in every head, 64 caller rows spread over the last
    256 real rows, checked against the replay (strict), the reference bounded
    by its own bf16-vs-fp32-dequant gap on the same rows (every config,
    BLASST included), the reference's cosine (the dense configurations) and,
    for BLASST, the per-row skip counts (exact)."""
    from low_bit_fake_quant.attention_kernel import launch_attention
    from low_bit_fake_quant.wan import make_inputs, pad_qkv, workloads
    w = workloads()[config]
    cfg = w.cfg
    q, k, v = make_inputs(w, seed=0, heads=4)
    qp, kp, vp, n = pad_qkv(q, k, v, cfg)
    assert n == w.N and qp.shape[1] > n
    ops, sm = parity.kernel_operands(qp, kp, vp, cfg, gpu)
    bl = cfg.blasst_lambda is not None
    res = launch_attention(ops, cfg, sm, torch.bfloat16, return_row_skips=bl)
    out, rsk = res if bl else (res, None)
    out = out.cpu()
    rows = torch.randperm(ops.s, generator=torch.Generator().manual_seed(config))[:1024]
    caller, u, rep, ref, dbg_rep, ref32 = parity.sampled_rows(qp, kp, vp, cfg, ops, rows, sm, tail=64, n_real=n,
                                                              with_ref32=True)
    assert ((caller >= n - 256) & (caller < n)).sum(1).min() >= 64, "every head checks rows next to N"
    got = parity.gather_caller_rows(out, caller)
    alw = dbg_rep["flip_allowance"].permute(0, 2, 1, 3)
    parity.strict_check(got, rep, f"config {config}", allowance=alw)
    # padding rows (Q zero rows past N) are sliced off by the caller
    real = (caller < n).reshape(ops.b, ops.h, -1).permute(0, 2, 1)[..., None].expand_as(got)
    keep = lambda t: torch.where(real, t.float(), torch.zeros((), dtype=torch.float32))  # noqa: E731
    st = parity.reference_bound(keep(got), keep(ref), keep(ref32), keep(rep), f"config {config}", allowance=alw)
    print(f"config {config}: S={qp.shape[1]} heads={ops.h} rows={caller.shape[1]} {st}")
    if bl:
        got_skips = torch.gather(rsk.cpu(), 1, caller)
        assert torch.equal(got_skips, dbg_rep["row_skips"].reshape(ops.b * ops.h, -1))
        print(f"config {config}: skip rate of the sample {got_skips.sum() / (got_skips.numel() * ops.s / 64):.3f}")
    elif st["ref_self_cos"] >= COS_MIN:
        assert st["cos_ref"] >= COS_MIN, f"config {config}: vs reference cos={st['cos_ref']:.7f}"
    else:
        # the reference itself misses 0.9999 against its exact-dequant variant on
        # this sample: its own bf16 rounding of the dequantised Q/K is the gap, and
        # the angle bound in reference_bound holds the kernel to it
        print(f"config {config}: the reference's own bf16-vs-fp32 cosine {st['ref_self_cos']:.7f} < {COS_MIN}")


@pytest.mark.parametrize("v_kind", [0, 2])
def test_v_tile_colsum_matches_decoded_sums(gpu, v_kind):
    """lbfq_v_tile_colsum: per 64-key tile, the column sums of the decoded V^T
    codes (MX: times 2^(e-127) of the key block), against a float64 sum of the
    oracle's E4M3 decode, within fp32 summation error; S ragged (partial last
    tile sums only its valid keys)."""
    import numpy as np

    from low_bit_fake_quant.attention_kernel import v_tile_colsum
    from oracle import fp8
    g = torch.Generator().manual_seed(5 + v_kind)
    b, h, d, P, s = 1, 3, 128, 384, 320 if v_kind == 2 else 300
    codes = torch.randint(0, 256, (b, h, d, P), generator=g, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes (the quantisers never write them)
    vb = 64
    ve = torch.randint(120, 135, (b, h, s // vb, d), generator=g, dtype=torch.uint8)
    out = v_tile_colsum(codes.to(gpu), ve.to(gpu), v_kind, vb, s).cpu().double()
    val = torch.from_numpy(fp8.decode(codes.numpy()).astype(np.float64))  # (b,h,d,P)
    nt = (s + 63) // 64
    for t in range(nt):
        k0, k1 = 64 * t, min(64 * t + 64, s)
        want = val[..., k0:k1].sum(-1)                       # (b,h,d)
        mag = val[..., k0:k1].abs().sum(-1)
        if v_kind == 2:
            sc = torch.pow(2.0, ve[:, :, k0 // vb, :].double() - 127)
            want, mag = want * sc, mag * sc
        got = out.view(b, h, -1, d)[:, :, t]
        assert ((got - want).abs() <= mag * 2.0 ** -21 + 1e-30).all(), t


def test_blasst_elided_tiles_match_the_mfma_path(gpu):
    """Tiles that every row of a wave skips are applied as fill x V column
    sums (no softmax, no rescale, zero P codes for the next PV).  With and
    without the column-sum table (every tile through the PV MFMAs) the output
    meets the strict bound against the reference algorithm replayed on the
    kernel's scores, and some tiles were elided.  (The two differ by fp32
    reassociation and by the FP8 MFMA's accumulation error, which the fp32
    column sums do not have.)"""
    from low_bit_fake_quant.attention_kernel import launch_attention
    for fill, p_quant in (("mean_a1.5", "dynamic"), ("max", "elementwise"), ("thr_a0.25", "mx")):
        cfg = _cfg(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                   q_kmeans_k=16, p_quant=p_quant, p_mx_block_n=64,
                   rowmax_mode="qm_k" if p_quant == "dynamic" else "online", blasst_lambda=0.05, blasst_fill=fill)
        q, k, v = _inputs(n=1024, seed=21, field=(4, 16, 16))
        ops, sm = parity.kernel_operands(q, k, v, cfg, gpu)
        assert ops.v_colsum is not None
        out, wt = launch_attention(ops, cfg, sm, torch.bfloat16, return_wave_tiles=True)
        ref = launch_attention(dataclasses.replace(ops, v_colsum=None), cfg, sm, torch.bfloat16)
        assert wt[..., 0].sum() > 0, "test input should make whole waves skip"
        u = parity.kernel_scores(ops, cfg, sm)
        rep, dbg = parity.replay(q, k, v, cfg, ops, u)
        alw = dbg["flip_allowance_nhd"]
        parity.strict_check(out.cpu(), rep, f"elided-{fill}", allowance=alw)
        parity.strict_check(ref.cpu(), rep, f"mfma-{fill}", allowance=alw)
        d = (out.float() - ref.float()).abs()
        print(f"{fill}/{p_quant}: elided wave tiles {int(wt[..., 0].sum())}, elided vs MFMA path max|diff| "
              f"{d.max().item():.3e}, {int((d > 0).sum())} of {d.numel()} outputs differ")


BATCH_CASES = {
    "dense_qmk_kmeans": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                             q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k"),
    "dense_online": dict(qk_quant="fp8_block", fp8_block_size=128, v_quant="fp8_channel", smoothing="full",
                         q_smooth_block_size=128, q_kmeans_k=None, p_quant="dynamic"),
    "blasst_mean_elided": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                               q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05,
                               blasst_fill="mean_a1.5"),
    "blasst_uta16": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                         q_kmeans_k=16, p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05,
                         blasst_fill="uta16_a1.5"),
    "blasst_block128_mx": dict(qk_quant="mxfp8", v_quant="mxfp8", v_mxfp8_block_size=128, smoothing="k_only",
                               q_kmeans_k=None, p_quant="mx", p_mx_block_n=128, p_requant_block_n=128,
                               blasst_lambda=0.05, blasst_fill="logn"),
}


@pytest.mark.parametrize("name", sorted(BATCH_CASES))
def test_batch_of_two_matches_oracle(gpu, name):
    """B = 2 with different inputs per batch entry: every per-(batch, head)
    table (Q/K/V codes and scales, permutations, qmk bias, V column sums,
    BLASST counters) is indexed by b*H + h; the pair must meet the strict
    bound against the replay, and each entry must equal the same configuration
    run on that entry alone bit for bit.  (With k-means the centroid seeds
    are drawn per slice index b*H + h, so only entry 0 shares its seeds with a
    single run.)"""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**BATCH_CASES[name])
    parts = [_inputs(n=1024, seed=30 + i, q_clusters=4, v_bias=True, field=(4, 16, 16)) for i in range(2)]
    q, k, v = (torch.cat([p[j] for p in parts], 0) for j in range(3))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    check_parity(out, q, k, v, cfg, f"batch2-{name}")
    for i, (qi, ki, vi) in enumerate(parts):
        if i > 0 and cfg.q_kmeans_k is not None:
            continue
        one = fake_quant_attention(qi.to(gpu), ki.to(gpu), vi.to(gpu), cfg).cpu()
        assert torch.equal(one, out[i:i + 1]), f"{name}: batch entry {i} differs from its single run"


@pytest.mark.parametrize("n", [1, 17, 63, 65, 129])
@pytest.mark.parametrize("blasst", [False, True])
def test_tiny_and_odd_sequence_lengths(gpu, n, blasst):
    """S below one 64-key tile, one key past a tile, one tile past the
    128-query workgroup: a single masked tile, the ring prefetch clamped to the
    last tile, and a workgroup whose second wave holds no valid query.  MX Q/K
    and channel V accept any S."""
    from low_bit_fake_quant import fake_quant_attention
    kw = dict(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="k_only", q_kmeans_k=None,
              p_quant="dynamic", rowmax_mode="online")
    if blasst:
        kw.update(blasst_lambda=0.05, blasst_fill="mean_a1.5")
    cfg = _cfg(**kw)
    q, k, v = _inputs(n=n, seed=40 + n, q_clusters=0)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    assert out.shape == q.shape and torch.isfinite(out).all()
    check_parity(out, q, k, v, cfg, f"S={n}{'/blasst' if blasst else ''}")


EIGHT_WAVE_CASES = {
    "elementwise_online_konly": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel",
                                     smoothing="k_only", q_kmeans_k=None, p_quant="elementwise"),
    "dynamic_online_full": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="full",
                                q_smooth_block_size=64, q_kmeans_k=None, p_quant="dynamic"),
    "dynamic_qmk_kmeans": dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="full",
                               q_smooth_block_size=64, q_kmeans_k=4, p_quant="dynamic", rowmax_mode="qm_k"),
}


@pytest.mark.parametrize("n", [64, 320, 960])
@pytest.mark.parametrize("name", sorted(EIGHT_WAVE_CASES))
def test_eight_wave_workgroups_ragged(gpu, name, n):
    """Dense fp8_block Q/K at D = 128 without V smoothing runs 256-query
    (eight-wave) workgroups.  S = 64, 320 and 960 leave the last workgroup
    with 64, 64 and 192 valid queries of 256: six, six and two of its waves
    hold no valid query but still stage their share of every K/V tile and
    meet every barrier.  One case per row-max mode (online, online + Q-smoothing bias,
    qm_k estimate) and P mode (elementwise, dynamic)."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**EIGHT_WAVE_CASES[name])
    q, k, v = _inputs(n=n, seed=50 + n, q_clusters=4 if n >= 256 else 0, v_bias=True)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    assert out.shape == q.shape and torch.isfinite(out).all()
    check_parity(out, q, k, v, cfg, f"8w-{name}-S={n}")
