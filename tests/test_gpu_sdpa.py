"""Path A (``p_requant=False``, reference attention.py:245-321): the native
SDPA kernels (lbfq_sdpa_dequant, lbfq_sdpa_fwd) against the CPU oracle.

* operands: the Q, K and V^T that lbfq_sdpa_dequant writes in the SDPA dtype
  equal the oracle's dequantised tensors (attention.py:274-286, V block means
  added in that dtype) bit for bit; the padding rows / keys are zero;
* attention: the output equals the reference's attention (attention.py:
  288-319) evaluated in float64 on the kernel's own operands, element-wise
  within one SDPA-dtype ulp of the value plus what the kernel's fp32
  arithmetic can legitimately move (``parity.sdpa_replay``): the main score's
  rounding to the SDPA dtype and P's rounding where the float64 value lies
  within the fp32 error of a rounding boundary (Q-smoothing branch), the
  fp32 score / P error (no-qm branch, P kept to ~16 bits);
* end to end: cosine >= 0.9999 and max |diff| <= 1e-2 against the oracle's
  SDPA path (which runs the reference's formulas on the CPU), including
  ragged S, fp16 and fp32 inputs, Hadamard, k-means and both smoothings.
"""

import pytest
import torch

import parity
from conftest import cosine, cpu_randn, max_abs
from oracle import pipeline as opipe

pytestmark = pytest.mark.gpu


def _cfg(**kw):
    from low_bit_fake_quant import QuantConfig
    base = dict(p_requant=False)
    base.update(kw)
    return QuantConfig(**base)


def _inputs(h=2, n=512, d=128, seed=0, q_clusters=0, v_bias=False, dtype=torch.bfloat16):
    from low_bit_fake_quant.wan import Workload, make_inputs
    w = Workload("t", h, n, d, None, q_clusters=q_clusters, v_bias=v_bias)
    return make_inputs(w, seed=seed, dtype=dtype)


CASES = {
    # name: (cfg, input kwargs)
    "plain_fp8block_channelV": (dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel",
                                     smoothing="off", q_kmeans_k=None, v_smooth_mode="off"), dict(n=512, d=128)),
    "konly_mx_ragged": (dict(qk_quant="mxfp8", mxfp8_block_size=32, v_quant="mxfp8", v_mxfp8_block_size=8,
                             smoothing="k_only", q_kmeans_k=None, v_smooth_mode="off"), dict(n=1000, d=64)),
    "tiny_s40": (dict(qk_quant="fp8_block", fp8_block_size=8, v_quant="fp8_block", v_fp8_block_size=8,
                      smoothing="off", q_kmeans_k=None, v_smooth_mode="off"), dict(n=40, d=128)),
    "full_kmeans_hadamard_vsmooth": (dict(smoothing="full", q_smooth_block_size=128, q_kmeans_k=8, qk_hadamard=True,
                                          v_smooth_mode="per_block", v_smooth_block_size=64),
                                     dict(n=512, d=64, q_clusters=4)),
    "full_fp16_blockV": (dict(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_block", v_fp8_block_size=128,
                              smoothing="full", q_smooth_block_size=64, q_kmeans_k=None, v_smooth_mode="off"),
                         dict(n=768, d=128, dtype=torch.float16, v_bias=True)),
    "full_group48_mx_vsmooth": (dict(qk_quant="mxfp8", mxfp8_block_size=32, v_quant="mxfp8", v_mxfp8_block_size=32,
                                     smoothing="full", q_smooth_block_size=48, q_kmeans_k=None,
                                     v_smooth_mode="per_block", v_smooth_block_size=96),
                                dict(n=480, d=128, v_bias=True)),
    "full_fp32_in_kmeans": (dict(qk_quant="fp8_block", fp8_block_size=32, v_quant="fp8_channel", smoothing="full",
                                 q_smooth_block_size=256, q_kmeans_k=16, v_smooth_mode="off"),
                            dict(n=1024, d=128, dtype=torch.float32, q_clusters=8)),
    # fp16 inputs through the Hadamard rotation: the rotated value is the fp32
    # product rounded to fp16 (the reference's two roundings), then quantised
    "fp16_hadamard_mx_full": (dict(qk_quant="mxfp8", mxfp8_block_size=32, qk_hadamard=True, v_quant="mxfp8",
                                   v_mxfp8_block_size=64, smoothing="full", q_smooth_block_size=128,
                                   q_kmeans_k=None, v_smooth_mode="per_block", v_smooth_block_size=64),
                              dict(n=640, d=128, dtype=torch.float16, v_bias=True)),
    "fp16_hadamard_block_konly": (dict(qk_quant="fp8_block", fp8_block_size=64, qk_hadamard=True,
                                       v_quant="fp8_channel", smoothing="k_only", q_kmeans_k=None,
                                       v_smooth_mode="off"),
                                  dict(n=512, d=64, dtype=torch.float16)),
}


def _operands(q, k, v, cfg, dev):
    from low_bit_fake_quant.attention import _lazy_preprocess, sdpa_operands
    sm = q.shape[-1] ** -0.5
    sdpa_dtype = torch.float16 if q.dtype == torch.float16 else torch.bfloat16
    prep = _lazy_preprocess(q.to(dev), k.to(dev), v.to(dev), cfg)
    return sdpa_operands(prep, cfg, sm, sdpa_dtype), sm, sdpa_dtype


def _bits(t):
    return t.contiguous().view(torch.int16)


def _assert_bits_equal(got, want, what):
    bad = (_bits(got) != _bits(want)).nonzero()
    if len(bad):
        ex = [(tuple(i.tolist()), got[tuple(i)].item(), want[tuple(i)].item()) for i in bad[:6]]
        raise AssertionError(f"{what}: {len(bad)} of {got.numel()} elements differ, e.g. {ex}")


@pytest.mark.parametrize("name", list(CASES))
def test_operands_equal_oracle_dequant(gpu, name):
    cfg = _cfg(**CASES[name][0])
    q, k, v = _inputs(**CASES[name][1], seed=3)
    sops, sm, dt = _operands(q, k, v, cfg, gpu)
    s = q.shape[1]
    q_work, k_work, v_work, qm, v_alpha, _, _ = opipe.preprocess(q, k, v, cfg)
    qi, ki = opipe.qk_quant_inputs(q_work, k_work, cfg)
    perm = (0, 2, 1, 3)
    for name_t, src, got in (("q", qi, sops.q), ("k", ki, sops.k)):
        c, sc, meta = opipe.quant_qk(src, cfg)
        want = opipe.dequant_qk(c, sc, meta, dt).permute(*perm).contiguous()
        got = got.cpu()
        _assert_bits_equal(got[:, :, :s], want, f"{name}: {name_t}")
        assert not got[:, :, s:].any(), f"{name}: {name_t} padding rows not zero"
    vc, vs, vmeta = opipe.quant_v(v_work, cfg)
    v_deq = opipe.dequant_v(vc, vs, vmeta, dt)
    if v_alpha is not None:
        v_deq = v_deq + v_alpha.repeat_interleave(cfg.v_smooth_block_size, dim=1).to(dt)
    want = v_deq.permute(0, 2, 3, 1).contiguous()  # (B,H,D,S)
    got = sops.v_t.cpu()
    _assert_bits_equal(got[..., :s], want, f"{name}: V^T")
    assert not got[..., s:].any(), f"{name}: V^T padding keys not zero"


@pytest.mark.parametrize("name", list(CASES))
def test_attention_equals_float64_replay(gpu, name):
    from low_bit_fake_quant.attention import launch_sdpa
    cfg = _cfg(**CASES[name][0])
    q, k, v = _inputs(**CASES[name][1], seed=5)
    sops, sm, dt = _operands(q, k, v, cfg, gpu)
    out = launch_sdpa(sops, sm, q.dtype)
    st = parity.sdpa_replay(sops, out, sm)
    print(f"{name}: {st}")
    assert st["excess"] <= 1.0, f"{name}: {st}"
    assert st["frac_equal"] >= 0.97, f"{name}: {st}"


@pytest.mark.parametrize("name", list(CASES))
def test_end_to_end_matches_oracle(gpu, name):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES[name][0])
    q, k, v = _inputs(**CASES[name][1], seed=7)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    assert out.dtype == q.dtype and out.shape == q.shape
    c, m = cosine(out, ref), max_abs(out, ref)
    print(f"{name}: cos={c:.7f} max_abs={m:.3e}")
    assert c >= parity.COS_MIN and m <= parity.MAXABS, f"{name}: cos={c:.7f} maxabs={m:.3e}"


def test_fp32_input_output_is_sdpa_rounded(gpu):
    """fp32 inputs: the output holds SDPA-dtype (bf16) values stored as fp32,
    as the reference's ``.to(out_dtype)`` of a bf16 result."""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES["plain_fp8block_channelV"][0])
    q, k, v = _inputs(n=256, d=64, seed=9, dtype=torch.float32)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg)
    assert out.dtype == torch.float32
    assert torch.equal(out, out.to(torch.bfloat16).float())


def test_sdpa_rejects_bad_arguments(gpu):
    from low_bit_fake_quant import _lib
    from low_bit_fake_quant.attention import launch_sdpa
    cfg = _cfg(**CASES["plain_fp8block_channelV"][0])
    q, k, v = _inputs(n=256, d=64, seed=9)
    sops, sm, dt = _operands(q, k, v, cfg, gpu)
    p = _lib.SdpaParams(B=1, H=2, S=256, D=96, s_pitch=256, q=sops.q.data_ptr(), k=sops.k.data_ptr(),
                        v_t=sops.v_t.data_ptr(), sdpa_dtype=2, sm_scale=sm, out=sops.q.data_ptr(), out_dtype=2)
    with pytest.raises(ValueError, match="D must be 64 or 128"):
        _lib.check(_lib.load().lbfq_sdpa_fwd(p, _lib.stream_handle(gpu)), "lbfq_sdpa_fwd")
    p.D, p.s_pitch = 64, 200
    with pytest.raises(ValueError, match="multiple of 128"):
        _lib.check(_lib.load().lbfq_sdpa_fwd(p, _lib.stream_handle(gpu)), "lbfq_sdpa_fwd")
    p.s_pitch, p.sdpa_dtype = 256, 0
    with pytest.raises(ValueError, match="bf16 or fp16"):
        _lib.check(_lib.load().lbfq_sdpa_fwd(p, _lib.stream_handle(gpu)), "lbfq_sdpa_fwd")
    out = launch_sdpa(sops, sm, torch.bfloat16)  # the valid call still works
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("name", ["full_kmeans_hadamard_vsmooth", "konly_mx_ragged"])
def test_batch_of_two(gpu, name):
    """B = 2 with different inputs per batch entry: each entry equals its own
    single-entry call bit for bit, and the whole output matches the oracle.
    (With k-means the centroid seeds are drawn per slice index b*H + h, so
    only entry 0 shares its seeds with a single run.)"""
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg(**CASES[name][0])
    parts = [_inputs(**CASES[name][1], seed=s) for s in (21, 22)]
    q, k, v = (torch.cat([p[j] for p in parts], 0) for j in range(3))
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    for i, p in enumerate(parts):
        if i > 0 and cfg.q_kmeans_k is not None:
            continue
        one = fake_quant_attention(*(t.to(gpu) for t in p), cfg).cpu()
        assert torch.equal(one, out[i:i + 1]), f"{name}: batch entry {i} differs from its single run"
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    c, m = cosine(out, ref), max_abs(out, ref)
    assert c >= parity.COS_MIN and m <= parity.MAXABS, f"{name}: cos={c:.7f} maxabs={m:.3e}"


@pytest.mark.timeout(600)
@pytest.mark.parametrize("config", [1, 2])
def test_full_length_wan_shapes_sampled_rows(gpu, config):
    """BASELINE configs 1 and 2 with p_requant=False at full length (2 heads,
    N = 32760 padded to 32768): the float64 replay on 1024 sampled kernel rows
    of each head, 64 of them within 256 of N, within the element-wise bound."""
    import dataclasses
    from low_bit_fake_quant.attention import launch_sdpa
    from low_bit_fake_quant.wan import make_inputs, pad_qkv, workloads
    w = workloads()[config]
    cfg = dataclasses.replace(w.cfg, p_requant=False)
    q, k, v = make_inputs(w, seed=0, heads=2)
    q, k, v, n = pad_qkv(q, k, v, cfg)
    sops, sm, dt = _operands(q, k, v, cfg, gpu)
    out = launch_sdpa(sops, sm, q.dtype)
    s = q.shape[1]
    g = torch.Generator().manual_seed(4)
    # caller rows: random ones and 64 within 256 of N; per head in kernel order
    caller = torch.cat([torch.randperm(s, generator=g)[:960], torch.linspace(n - 256, s - 1, 64).long()])
    if sops.out_row_map is None:
        rows = caller
    else:
        inv = torch.argsort(sops.out_row_map.cpu().long(), dim=1)   # output row -> kernel row
        rows = inv[:, caller]
    st = parity.sdpa_replay(sops, out, sm, rows=rows)
    print(f"config {config}: {st}")
    assert st["excess"] <= 1.0, f"config {config}: {st}"
    assert st["frac_equal"] >= 0.97, f"config {config}: {st}"


@pytest.mark.parametrize("d,dtype", [(64, torch.bfloat16), (128, torch.bfloat16), (128, torch.float16)])
@pytest.mark.parametrize("qm", [False, True])
def test_eight_wave_workgroups_past_the_pitch(gpu, qm, d, dtype):
    """Eight-wave (256-query) workgroups, used when there are at least 256 of
    them, with a pitch that is an odd multiple of 128 (S = 21888, 3 heads:
    258 workgroups, the last one's upper half past the pitch), at both head
    dims (one 16-byte K and one V^T chunk per thread per tile at D = 64, two
    at D = 128), bf16 and fp16: the float64 replay on 1024 sampled rows of
    each head, 128 of them the last rows."""
    from low_bit_fake_quant.attention import launch_sdpa
    s, h = 21888, 3
    kw = dict(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="full" if qm else "k_only", q_kmeans_k=None,
              v_smooth_mode="off", q_smooth_block_size=128)
    cfg = _cfg(**kw)
    q, k, v = (cpu_randn(1, s, h, d, seed=sd, scale=1.5, dtype=dtype) for sd in (31, 32, 33))
    sops, sm, dt = _operands(q, k, v, cfg, gpu)
    assert sops.P == s and (s // 128) % 2 == 1 and h * ((s + 255) // 256) >= 256
    out = launch_sdpa(sops, sm, q.dtype)
    g = torch.Generator().manual_seed(6)
    rows = torch.cat([torch.randperm(s - 128, generator=g)[:896], torch.arange(s - 128, s)])
    st = parity.sdpa_replay(sops, out, sm, rows=rows)
    assert st["excess"] <= 1.0, st
    assert st["frac_equal"] >= 0.97, st


@pytest.mark.parametrize("n", [1, 3, 17, 65, 129])
@pytest.mark.parametrize("qm", [False, True])
def test_tiny_and_odd_sequence_lengths(gpu, n, qm):
    """S below one 64-key tile, one key past a tile, one row past the
    128-query workgroup (waves of padding rows only); with Q smoothing, groups
    of one row (n = 1) or of the whole sequence.  MX Q/K and channel V accept
    any S."""
    from low_bit_fake_quant import fake_quant_attention
    from low_bit_fake_quant.attention import launch_sdpa
    kw = dict(qk_quant="mxfp8", v_quant="fp8_channel", smoothing="full" if qm else "k_only", q_kmeans_k=None,
              v_smooth_mode="off")
    if qm:
        kw["q_smooth_block_size"] = 1 if n == 1 else n
    cfg = _cfg(**kw)
    q, k, v = _inputs(n=n, d=64, seed=50 + n)
    out = fake_quant_attention(q.to(gpu), k.to(gpu), v.to(gpu), cfg).cpu()
    assert out.shape == q.shape and torch.isfinite(out.float()).all()
    ref = opipe.fake_quant_attention(q, k, v, cfg)
    c, m = cosine(out, ref), max_abs(out, ref)
    assert c >= parity.COS_MIN and m <= parity.MAXABS, f"S={n}: cos={c:.7f} maxabs={m:.3e}"
    sops, sm, _ = _operands(q, k, v, cfg, gpu)
    st = parity.sdpa_replay(sops, launch_sdpa(sops, sm, q.dtype), sm)
    assert st["excess"] <= 1.0, f"S={n}: {st}"
