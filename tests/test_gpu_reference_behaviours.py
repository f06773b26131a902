"""The behaviours the reference's own test suite asserts about the public API,
held by this build on the GPU (same entry points, configurations, shapes and
thresholds; inputs drawn from seeded CPU generators instead of CUDA ones).

Sources: tests/test_fake_quant_attention.py:38-125, test_qk_hadamard.py:13-94,
test_v_kmeans.py:39-133, test_v_smoothing.py:51-137 and
test_v_quant_variants.py:37-173 of the reference.  The reference's
kernel-level tests (test_triton_attn.py, test_v_smoothing.py:139-183) are
held by tests/test_gpu_attention_triton.py.
"""

import itertools

import pytest
import torch

pytestmark = pytest.mark.gpu


def _qkv(gpu, b=1, s=512, h=2, d=64, seed=0, dtype=torch.bfloat16, v_block_bias=0.0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, s, h, d, generator=g) for _ in range(3))
    if v_block_bias:
        # a strong per-block bias of V over 8 blocks of S, so V smoothing matters
        nb = 8
        bias = torch.randn(b, nb, 1, h, d, generator=g) * v_block_bias
        v = (v.view(b, nb, s // nb, h, d) + bias).view(b, s, h, d)
    return tuple(t.to(dtype).to(gpu) for t in (q, k, v))


def _cos(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return (a @ b / (a.norm() * b.norm())).item()


def _mse(a, b):
    return (a.float() - b.float()).pow(2).mean().item()


def _cfg(**kw):
    from low_bit_fake_quant import QuantConfig
    return QuantConfig(**kw)


# ---- test_fake_quant_attention.py ------------------------------------------

@pytest.mark.parametrize("qk_quant,smoothing,kmeans_k,p_requant",
                         list(itertools.product(["fp8_block", "mxfp8"], ["off", "k_only", "full"], [None, 32],
                                                [False, True])))
def test_runs_and_tracks_exact_attention(gpu, qk_quant, smoothing, kmeans_k, p_requant):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    cfg = _cfg(qk_quant=qk_quant, v_quant="fp8_channel", smoothing=smoothing, q_kmeans_k=kmeans_k,
               q_smooth_block_size=128, fp8_block_size=128, mxfp8_block_size=32, p_requant=p_requant,
               p_requant_q_chunk=128)
    q, k, v = _qkv(gpu)
    o = fake_quant_attention(q, k, v, cfg)
    assert o.shape == q.shape and torch.isfinite(o).all()
    c = _cos(o, reference_attention(q, k, v))
    assert c > 0.93, f"cos={c:.4f}"


def test_p_requant_and_sdpa_paths_agree(gpu):
    from low_bit_fake_quant import fake_quant_attention
    base = dict(qk_quant="fp8_block", smoothing="off", q_kmeans_k=None, q_smooth_block_size=128)
    q, k, v = _qkv(gpu, s=256, seed=7)
    o_a = fake_quant_attention(q, k, v, _cfg(**base, p_requant=False))
    o_b = fake_quant_attention(q, k, v, _cfg(**base, p_requant=True, p_requant_q_chunk=128))
    assert _cos(o_a, o_b) > 0.99


@pytest.mark.parametrize("fill", ["mean_a1.5", "uta16_a1.5"])
def test_blasst_fills_run(gpu, fill):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", v_quant="fp8_channel", smoothing="off", q_kmeans_k=None,
               q_smooth_block_size=128, fp8_block_size=128, p_requant=True, p_requant_block_m=64,
               p_requant_block_n=64, blasst_lambda=0.8, blasst_fill=fill)
    q, k, v = _qkv(gpu, s=256, seed=13)
    o = fake_quant_attention(q, k, v, cfg)
    assert o.shape == q.shape and torch.isfinite(o).all()


def test_blasst_needs_p_requant(gpu):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", smoothing="off", q_kmeans_k=None, q_smooth_block_size=128, p_requant=False,
               blasst_lambda=0.8, blasst_fill="mean_a1.5")
    q, k, v = _qkv(gpu, s=256, seed=14)
    with pytest.raises(ValueError, match="requires cfg.p_requant=True"):
        fake_quant_attention(q, k, v, cfg)


# ---- test_qk_hadamard.py ----------------------------------------------------

def test_hadamard_keeps_unquantised_logits(gpu):
    from low_bit_fake_quant import apply_qk_hadamard
    q, k, _ = _qkv(gpu, s=128, dtype=torch.float32)
    qr, kr = apply_qk_hadamard(q, k, random_sign=True, seed=123)
    logits = lambda a, b: torch.matmul(a.permute(0, 2, 1, 3), b.permute(0, 2, 3, 1).contiguous())  # noqa: E731
    assert (logits(qr, kr) - logits(q, k)).abs().max().item() < 2e-4


def test_hadamard_cuts_fp8_block_score_error(gpu):
    """One channel carries a +-30 trend (opposite signs in Q and K); rotating
    spreads it over D, so the fp8_block scores get at least 4x closer."""
    from low_bit_fake_quant.attention import _dequant_qk, _qk_inputs_for_quant, _quant_qk
    s = 256
    q, k, _ = _qkv(gpu, s=s, seed=1)
    q, k = q * 0.2, k * 0.2
    trend = torch.linspace(-30, 30, s, dtype=torch.bfloat16, device=gpu).view(1, s, 1)
    q[..., 0] += trend
    k[..., 0] -= trend

    def score_mse(cfg):
        qi, ki = _qk_inputs_for_quant(q, k, cfg)
        qd = _dequant_qk(*_quant_qk(qi, cfg), torch.bfloat16)
        kd = _dequant_qk(*_quant_qk(ki, cfg), torch.bfloat16)
        mm = lambda a, b: torch.matmul(a.permute(0, 2, 1, 3).float(), b.permute(0, 2, 3, 1).float())  # noqa: E731
        return (mm(qd, kd) - mm(q, k)).square().mean().item()

    base = dict(qk_quant="fp8_block", smoothing="off", q_kmeans_k=None, v_smooth_mode="off", p_requant=False)
    assert score_mse(_cfg(**base, qk_hadamard=True, qk_hadamard_seed=0)) < 0.25 * score_mse(_cfg(**base))


@pytest.mark.parametrize("p_requant", [False, True])
def test_hadamard_runs_with_smoothing_off(gpu, p_requant):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="fp8_block", v_quant="fp8_channel", smoothing="off", q_kmeans_k=None, v_smooth_mode="off",
               v_kmeans_k=None, qk_hadamard=True, p_requant=p_requant, p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu, s=256, seed=2)
    o = fake_quant_attention(q, k, v, cfg)
    assert o.shape == q.shape and torch.isfinite(o).all()


# ---- test_v_kmeans.py -------------------------------------------------------

def test_co_permuted_kv_keeps_exact_attention(gpu):
    from low_bit_fake_quant import apply_kv_permutation, reference_attention, v_kmeans_reorder
    q, k, v = _qkv(gpu)
    r = v_kmeans_reorder(v, n_clusters=32, max_iters=10, seed=0)
    o1 = reference_attention(q, k, v)
    o2 = reference_attention(q, apply_kv_permutation(k, r.order), r.tensor_reordered)
    assert _cos(o1, o2) > 0.9999
    assert (o1.float() - o2.float()).abs().max().item() < 1e-2


@pytest.mark.parametrize("p_requant,bound", [(False, 0.95), (True, 0.93)])
def test_v_kmeans_stack_tracks_exact_attention(gpu, p_requant, bound):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    cfg = _cfg(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="full", q_smooth_block_size=128, q_kmeans_k=32,
               v_smooth_mode="per_block", v_smooth_block_size=64, v_kmeans_k=32, p_requant=p_requant,
               p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu)
    o = fake_quant_attention(q, k, v, cfg)
    assert o.shape == q.shape and torch.isfinite(o).all()
    assert _cos(o, reference_attention(q, k, v)) > bound


def test_v_kmeans_helps_with_clustered_v(gpu):
    """V made of 8 clusters of very different magnitude, shuffled along S."""
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    g = torch.Generator().manual_seed(0)
    b, s, h, d = 1, 1024, 2, 64
    q = torch.randn(b, s, h, d, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(b, s, h, d, generator=g).to(torch.bfloat16).to(gpu)
    mags = torch.tensor([0.1, 0.5, 1.0, 2.0, 5.0, 0.3, 1.5, 4.0]).view(8, 1, 1)
    centres = torch.randn(8, h, d, generator=g) * mags
    ids = torch.randint(0, 8, (s,), generator=g)
    v = (centres[ids] + 0.1 * torch.randn(s, h, d, generator=g)).unsqueeze(0).to(torch.bfloat16).to(gpu)
    base = dict(qk_quant="fp8_block", v_quant="fp8_channel", smoothing="off", q_kmeans_k=None,
                v_smooth_mode="per_block", v_smooth_block_size=64, p_requant=False)
    ref = reference_attention(q, k, v)
    mse_no = _mse(fake_quant_attention(q, k, v, _cfg(**base, v_kmeans_k=None)), ref)
    mse_vk = _mse(fake_quant_attention(q, k, v, _cfg(**base, v_kmeans_k=32)), ref)
    assert mse_vk <= 1.05 * mse_no, (mse_vk, mse_no)


# ---- test_v_smoothing.py ----------------------------------------------------

def test_smooth_v_per_block(gpu):
    from low_bit_fake_quant import smooth_v_per_block
    b, s, h, d, blk = 1, 512, 2, 64, 64
    _, _, v = _qkv(gpu, s=s)
    vc, alpha = smooth_v_per_block(v, block_s=blk)
    assert vc.shape == v.shape and alpha.shape == (b, s // blk, h, d) and alpha.dtype == torch.float32
    assert vc.float().view(b, s // blk, blk, h, d).mean(dim=2).abs().max().item() < 1e-2
    want = v.float().view(b, s // blk, blk, h, d).mean(dim=2)
    assert (alpha - want).abs().max().item() < 1e-3


@pytest.mark.parametrize("p_requant,bound", [(False, 0.97), (True, 0.95)])
def test_v_smoothing_tracks_exact_attention(gpu, p_requant, bound):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    cfg = _cfg(qk_quant="fp8_block", v_quant="fp8_channel", smoothing="off", q_kmeans_k=None,
               q_smooth_block_size=128, fp8_block_size=128, v_smooth_mode="per_block", v_smooth_block_size=64,
               p_requant=p_requant, p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu, v_block_bias=2.0)
    assert _cos(fake_quant_attention(q, k, v, cfg), reference_attention(q, k, v)) > bound


def test_v_smoothing_helps_under_block_bias(gpu):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    base = dict(qk_quant="fp8_block", v_quant="fp8_channel", smoothing="off", q_kmeans_k=None, p_requant=False)
    q, k, v = _qkv(gpu, v_block_bias=4.0)
    ref = reference_attention(q, k, v)
    mse_off = _mse(fake_quant_attention(q, k, v, _cfg(**base, v_smooth_mode="off")), ref)
    mse_on = _mse(fake_quant_attention(q, k, v, _cfg(**base, v_smooth_mode="per_block", v_smooth_block_size=64)),
                  ref)
    assert mse_on <= 1.05 * mse_off, (mse_on, mse_off)


# ---- test_v_quant_variants.py ----------------------------------------------

@pytest.mark.parametrize("v_quant,v_smooth,p_requant",
                         list(itertools.product(["fp8_channel", "fp8_block", "mxfp8"], ["off", "per_block"],
                                                [False, True])))
def test_v_quant_variants_track_exact_attention(gpu, v_quant, v_smooth, p_requant):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    cfg = _cfg(qk_quant="fp8_block", v_quant=v_quant, smoothing="off", q_kmeans_k=None, q_smooth_block_size=128,
               fp8_block_size=128, mxfp8_block_size=32, v_fp8_block_size=64, v_mxfp8_block_size=64,
               v_smooth_mode=v_smooth, v_smooth_block_size=64, p_requant=p_requant, p_requant_block_m=64,
               p_requant_block_n=64)
    q, k, v = _qkv(gpu)
    o = fake_quant_attention(q, k, v, cfg)
    assert o.shape == q.shape and torch.isfinite(o).all()
    assert _cos(o, reference_attention(q, k, v)) > 0.93


@pytest.mark.parametrize("v_quant", ["fp8_channel", "fp8_block", "mxfp8"])
def test_full_stack_tracks_exact_attention(gpu, v_quant):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    cfg = _cfg(qk_quant="mxfp8", v_quant=v_quant, smoothing="full", q_smooth_block_size=128, q_kmeans_k=16,
               fp8_block_size=128, mxfp8_block_size=32, v_fp8_block_size=64, v_mxfp8_block_size=64,
               v_smooth_mode="per_block", v_smooth_block_size=64, v_kmeans_k=16, p_requant=True,
               p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu)
    assert _cos(fake_quant_attention(q, k, v, cfg), reference_attention(q, k, v)) > 0.95


def test_auto_p_with_mx_v_runs(gpu):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(qk_quant="mxfp8", v_quant="mxfp8", smoothing="off", q_kmeans_k=None, v_smooth_mode="off",
               v_mxfp8_block_size=64, p_quant="auto", p_requant=True, p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu, s=256)
    assert torch.isfinite(fake_quant_attention(q, k, v, cfg)).all()


def test_auto_p_with_fp8_block_v_tracks_exact_attention(gpu):
    from low_bit_fake_quant import fake_quant_attention, reference_attention
    cfg = _cfg(qk_quant="mxfp8", v_quant="fp8_block", smoothing="off", q_kmeans_k=None, v_smooth_mode="off",
               v_fp8_block_size=64, p_quant="auto", p_requant=True, p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu, s=256)
    assert _cos(fake_quant_attention(q, k, v, cfg), reference_attention(q, k, v)) > 0.95


def test_qm_k_row_max_tracks_online_with_dynamic_p(gpu):
    from low_bit_fake_quant import fake_quant_attention
    base = dict(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="full", q_smooth_block_size=128, q_kmeans_k=16,
                p_quant="dynamic", p_requant=True, p_requant_block_m=64, p_requant_block_n=64)
    q, k, v = _qkv(gpu, seed=3)
    online = fake_quant_attention(q, k, v, _cfg(**base, rowmax_mode="online"))
    est = fake_quant_attention(q, k, v, _cfg(**base, rowmax_mode="qm_k"))
    assert _cos(est, online) > 0.9999
    assert (est.float() - online.float()).abs().max().item() < 5e-3
