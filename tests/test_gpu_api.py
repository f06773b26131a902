"""The public API around the hot path against the CPU oracle: the
PreprocessCache work tensors (attention.py:647-703), return_artifacts
(attention.py:797-805), reference_attention (attention.py:809-825) and the
legacy prepare_qkv pipeline (pipeline.py:42-110)."""

import pytest
import torch

from conftest import cpu_randn
from oracle import pipeline as opipe

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    from low_bit_fake_quant import QuantConfig
    return QuantConfig(**kw)


def _inputs(n=512, h=2, d=128, seed=0, dtype=torch.bfloat16):
    from low_bit_fake_quant.wan import Workload, make_inputs
    return make_inputs(Workload("t", h, n, d, None, q_clusters=8, v_bias=True), seed=seed, dtype=dtype)


CACHE_CFGS = {
    "full_qkmeans": dict(smoothing="full", q_smooth_block_size=128, q_kmeans_k=8),
    "everything": dict(smoothing="full", q_smooth_block_size=256, q_kmeans_k=16, v_kmeans_k=16,
                       v_smooth_mode="per_block", v_smooth_block_size=64),
    "k_only": dict(smoothing="k_only", q_kmeans_k=None),
}


@pytest.mark.parametrize("name", sorted(CACHE_CFGS))
def test_preprocess_cache_tensors_match_oracle(gpu, name):
    """prepare_for_attention's work tensors, means and k-means permutations
    are bitwise the oracle's _preprocess (attention.py:166-239)."""
    from low_bit_fake_quant import prepare_for_attention
    cfg = _cfg(**CACHE_CFGS[name])
    q, k, v = _inputs(seed=len(name))
    cache = prepare_for_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg)
    qw, kw, vw, qm, v_alpha, q_km, v_km = opipe.preprocess(q, k, v, cfg)
    assert torch.equal(cache.q_work.cpu(), qw)
    assert torch.equal(cache.k_work.cpu(), kw)
    assert torch.equal(cache.v_work.cpu(), vw)
    for got, want in ((cache.qm, qm), (cache.v_alpha, v_alpha)):
        assert (got is None) == (want is None)
        if want is not None:
            assert torch.equal(got.cpu().float(), want.float())
    for got, want in ((cache.q_kmeans, q_km), (cache.v_kmeans, v_km)):
        assert (got is None) == (want is None)
        if want is not None:
            assert torch.equal(got.order.cpu().long(), want["order"].long())
            assert torch.equal(got.inverse_order.cpu().long(), want["inverse_order"].long())
            assert torch.equal(got.labels.cpu().long(), want["labels"].long())
            assert torch.equal(got.tensor_reordered.cpu(), want["tensor_reordered"])
    assert (cache.smoothing, cache.q_kmeans_k, cache.v_kmeans_k) == (cfg.smoothing, cfg.q_kmeans_k, cfg.v_kmeans_k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_return_artifacts_fields(gpu, dtype):
    """FakeQuantArtifacts (attention.py:797-805): qm and the Q k-means result
    equal the oracle's; q_eff_dtype is the SDPA dtype of the input dtype."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(smoothing="full", q_smooth_block_size=128, q_kmeans_k=8, qk_hadamard=True, p_requant=True,
               p_quant="dynamic")
    q, k, v = _inputs(seed=7, dtype=dtype)
    out, art = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg, return_artifacts=True)
    _, _, _, qm, _, q_km, _ = opipe.preprocess(q, k, v, cfg)
    assert torch.equal(art.qm.cpu().float(), qm.float())
    assert torch.equal(art.kmeans.order.cpu().long(), q_km["order"].long())
    assert torch.equal(art.kmeans.inverse_order.cpu().long(), q_km["inverse_order"].long())
    assert art.q_eff_dtype == (torch.float16 if dtype == torch.float16 else torch.bfloat16)
    assert art.p_requant is True and art.qk_hadamard is True
    assert out.shape == q.shape and out.dtype == dtype


@pytest.mark.parametrize("d", [64, 128])
def test_reference_attention_matches_float64_softmax(gpu, d):
    """reference_attention (attention.py:809-825): unquantised attention;
    within one bf16 ulp (+1e-3 absolute) of a float64 softmax."""
    from low_bit_fake_quant import reference_attention
    q = cpu_randn(1, 300, 3, d, seed=1)
    k = cpu_randn(1, 300, 3, d, seed=2)
    v = cpu_randn(1, 300, 3, d, seed=3)
    out = reference_attention(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    s = torch.einsum("bqhd,bkhd->bhqk", q.double(), k.double()) / d ** 0.5
    ref = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, -1), v.double())
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 7)
    assert out.dtype == q.dtype and ((out.double() - ref).abs() <= ulp + 1e-3).all()
    with pytest.raises(ValueError, match="must be"):
        reference_attention(q[0].to(gpu), k[0].to(gpu), v[0].to(gpu))


PREP_CFGS = {
    "fp8_block_full_kmeans_channelV": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full",
                                           q_smooth_block_size=128, q_kmeans_k=8, v_quant="fp8_channel"),
    "mx_hadamard_mxV": dict(qk_quant="mxfp8", qk_hadamard=True, smoothing="k_only", q_kmeans_k=None,
                            v_quant="mxfp8", v_mxfp8_block_size=64),
    "blockV_off": dict(qk_quant="fp8_block", fp8_block_size=128, smoothing="off", q_kmeans_k=None,
                       v_quant="fp8_block", v_fp8_block_size=64),
}


@pytest.mark.parametrize("name", sorted(PREP_CFGS))
def test_prepare_qkv_matches_oracle(gpu, name):
    """pipeline.prepare_qkv: codes, scales, qm, k_mean and the k-means order
    bitwise the oracle's; the qm.K_s correction (fp32 einsum in the
    reference) within 2^-20 of sum |qm| |K_s| of the exact value."""
    from low_bit_fake_quant import prepare_qkv
    cfg = _cfg(**PREP_CFGS[name])
    q, k, v = _inputs(seed=len(name))
    got = prepare_qkv(q.to(gpu), k.to(gpu), v.to(gpu), cfg)
    want = opipe.prepare_qkv(q, k, v, cfg)
    for f in ("q", "k", "v"):
        assert torch.equal(getattr(got, f).cpu().view(torch.uint8), want[f]), f
    for f in ("q_scale", "k_scale", "v_scale"):
        assert torch.equal(getattr(got, f).cpu().float(), want[f].float()), f
    for f in ("qm", "k_mean"):
        assert (getattr(got, f) is None) == (want[f] is None), f
        if want[f] is not None:
            assert torch.equal(getattr(got, f).cpu().float(), want[f].float()), f
    assert (got.kmeans is None) == (want["kmeans"] is None)
    if want["kmeans"] is not None:
        assert torch.equal(got.kmeans.order.cpu().long(), want["kmeans"]["order"].long())
    assert (got.correction is None) == (want["correction"] is None)
    if want["correction"] is not None:
        assert got.correction.dtype == cfg.correction_dtype
        _, _, _, _, kw = _work_after_smoothing(q, k, v, cfg)
        bound = torch.einsum("bqhd,bshd->bqhs", want["qm"].double().abs(), kw.double().abs()) * 2.0 ** -20
        err = (got.correction.cpu().double() - want["correction"]).abs()
        tol = bound + (want["correction"].abs() * 2.0 ** -8 if cfg.correction_dtype != torch.float32 else 0)
        assert (err <= tol).all()
    with pytest.raises(ValueError, match="must live on CUDA"):
        prepare_qkv(q, k, v, cfg)


def _work_after_smoothing(q, k, v, cfg):
    from oracle import preprocess as opre
    k_work, k_mean = opre.smooth_k(k.contiguous())
    return None, None, None, k_mean, k_work
