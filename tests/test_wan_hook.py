"""Wan call boundary (``low_bit_fake_quant.wan_hook``) against the reference
hook's behaviour (``bench/wan_attention_hook.py:203-327``).

CPU tests: patching, the self/cross heuristic, dtype cast and ``q_scale``,
the exact-attention fallback (against a float64 softmax), the dump format
and its call selection.  GPU tests: the self-attention path equals
``fake_quant_attention`` on explicitly padded inputs, bit for bit, and the
comparison records.
"""

import math
import types

import pytest
import torch

from conftest import cpu_randn

from low_bit_fake_quant import QuantConfig
from low_bit_fake_quant import wan_hook
from low_bit_fake_quant.wan import pad_qkv


@pytest.fixture(autouse=True)
def _clean_state(monkeypatch):
    for name in ("WAN_ATTENTION_DUMP_DIR", "WAN_ATTENTION_DUMP_CALLS", "WAN_ATTENTION_DUMP_LIMIT",
                 "WAN_ATTENTION_COMPARE_SDPA", "WAN_ATTENTION_COMPARE_ONLINE_ROWMAX"):
        monkeypatch.delenv(name, raising=False)
    wan_hook.set_quant_cfg(wan_hook.NO_QUANT)
    yield
    wan_hook.set_quant_cfg(wan_hook.NO_QUANT)


def _softmax_attention_f64(q, k, v, scale):
    qb, kb, vb = (t.double().transpose(1, 2) for t in (q, k, v))
    w = torch.softmax(qb @ kb.transpose(-1, -2) * scale, dim=-1)
    return (w @ vb).transpose(1, 2)


def _cfg2():
    return QuantConfig(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="full",
                       q_smooth_block_size=256, q_kmeans_k=8, p_requant=True, p_quant="dynamic",
                       rowmax_mode="qm_k", p_requant_block_m=64, p_requant_block_n=64)


def test_install_hook_patches_the_three_names():
    am = types.ModuleType("stub_wan_attention")
    mm = types.ModuleType("stub_wan_model")
    am.attention = am.flash_attention = mm.flash_attention = object()
    wan_hook.install_hook(am, mm)
    wan_hook.install_hook(am, mm)  # idempotent
    assert am.attention is wan_hook.fake_or_sdpa_attention
    assert am.flash_attention is wan_hook.fake_or_sdpa_attention
    assert mm.flash_attention is wan_hook.fake_or_sdpa_attention


def test_install_hook_without_wan_raises_import_error():
    try:
        import wan  # noqa: F401
        pytest.skip("a wan package is installed")
    except ImportError:
        pass
    with pytest.raises(ImportError):
        wan_hook.install_hook()


def test_self_attention_heuristic():
    assert wan_hook.is_self_attention(1025, 1025)
    assert not wan_hook.is_self_attention(1024, 1024)
    assert not wan_hook.is_self_attention(32760, 512)


@pytest.mark.parametrize("lq,lk,kind", [(1100, 512, "cross-sdpa"), (1024, 1024, "cross-sdpa"),
                                        (1100, 1100, "self-sdpa")])
def test_exact_paths_on_cpu(lq, lk, kind):
    # cross-attention always, short "self" calls and NO_QUANT self-attention run exact attention
    if kind != "self-sdpa":
        wan_hook.set_quant_cfg(_cfg2())
    q = cpu_randn(1, lq, 2, 64, seed=1)
    k = cpu_randn(1, lk, 2, 64, seed=2)
    v = cpu_randn(1, lk, 2, 64, seed=3)
    out = wan_hook.fake_or_sdpa_attention(q, k, v)
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    ref = _softmax_attention_f64(q, k, v, 1.0 / math.sqrt(64))
    # float32 attention rounded once to bf16: within one bf16 rounding of the float64 result
    assert ((out.double() - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-6).all()
    log = wan_hook.get_call_log()
    assert [r["kind"] for r in log] == [kind]
    assert log[0]["Lq"] == lq and log[0]["Lk"] == lk and log[0]["H"] == 2 and log[0]["D"] == 64


def test_dtype_cast_q_scale_and_softmax_scale():
    q = cpu_randn(1, 300, 2, 64, seed=4, dtype=torch.float32)
    k = cpu_randn(1, 200, 2, 64, seed=5, dtype=torch.float32)
    v = cpu_randn(1, 200, 2, 64, seed=6, dtype=torch.float32)
    out = wan_hook.fake_or_sdpa_attention(q, k, v, q_scale=0.5, softmax_scale=0.3, dtype=torch.float16)
    assert out.dtype == torch.float16
    qh, kh, vh = (t.to(torch.float16) for t in (q, k, v))
    ref = _softmax_attention_f64(qh * 0.5, kh, vh, 0.3)
    assert ((out.double() - ref).abs() <= ref.abs() * 2.0 ** -10 + 1e-6).all()


def test_dump_format_and_selection(tmp_path, monkeypatch):
    monkeypatch.setenv("WAN_ATTENTION_DUMP_DIR", str(tmp_path))
    q, k, v = (cpu_randn(1, 16, 2, 8, seed=s) for s in (7, 8, 9))
    # default limit: only the first call is dumped
    for i in range(3):
        rec = {"kind": "self-fq", "i": i}
        wan_hook._maybe_dump_qkv(q, k, v, rec)
        wan_hook._log_call(rec)
    log = wan_hook.get_call_log()
    assert log[0]["dumped_qkv"].endswith("call_000.pt")
    assert "dumped_qkv" not in log[1] and "dumped_qkv" not in log[2]
    obj = torch.load(log[0]["dumped_qkv"], weights_only=True)
    assert set(obj) == {"query", "key", "value", "record"}
    assert torch.equal(obj["query"], q) and torch.equal(obj["value"], v)
    assert obj["record"]["kind"] == "self-fq"
    lq, lk, lv = wan_hook.load_qkv_dump(log[0]["dumped_qkv"])
    assert torch.equal(lk, k)
    # explicit call list
    wan_hook.set_quant_cfg(None)
    monkeypatch.setenv("WAN_ATTENTION_DUMP_CALLS", "1,2")
    for i in range(4):
        rec = {"i": i}
        wan_hook._maybe_dump_qkv(q, k, v, rec)
        wan_hook._log_call(rec)
    assert [("dumped_qkv" in r) for r in wan_hook.get_call_log()] == [False, True, True, False]


@pytest.mark.gpu
def test_hook_self_attention_matches_padded_call(gpu):
    from low_bit_fake_quant import fake_quant_attention
    cfg = _cfg2()
    n = 1100  # pads to 1280 (LCM 256)
    q = cpu_randn(1, n, 2, 128, seed=11).to(gpu)
    k = cpu_randn(1, n, 2, 128, seed=12).to(gpu)
    v = cpu_randn(1, n, 2, 128, seed=13).to(gpu)
    wan_hook.set_quant_cfg(cfg)
    out = wan_hook.fake_or_sdpa_attention(q, k, v)
    qp, kp, vp, _ = pad_qkv(q, k, v, cfg)
    assert qp.shape[1] == 1280
    ref = fake_quant_attention(qp, kp, vp, cfg)[:, :n]
    assert out.shape == q.shape and torch.equal(out, ref)
    rec = wan_hook.get_call_log()[0]
    assert rec["kind"] == "self-fq" and rec["pad"] == 180
    # against the oracle: pad, the reference algorithm (replayed on the kernel's
    # scores: strict; and with its own scores: cosine), slice
    # (bench/wan_attention_hook.py:249-294)
    import parity
    from oracle import pipeline as opipe
    qc, kc, vc = (t.cpu() for t in (qp, kp, vp))
    ops, sm = parity.kernel_operands(qc, kc, vc, cfg, gpu)
    rep, dbg = parity.replay(qc, kc, vc, cfg, ops, parity.kernel_scores(ops, cfg, sm))
    parity.strict_check(out.cpu(), rep[:, :n], "hook", allowance=dbg["flip_allowance_nhd"][:, :n])
    oref = opipe.fake_quant_attention(qc, kc, vc, cfg)[:, :n]
    assert parity.cosine(out.cpu(), oref) >= parity.COS_MIN


@pytest.mark.gpu
def test_hook_comparison_records(gpu, monkeypatch, tmp_path):
    monkeypatch.setenv("WAN_ATTENTION_COMPARE_SDPA", "1")
    monkeypatch.setenv("WAN_ATTENTION_COMPARE_ONLINE_ROWMAX", "1")
    monkeypatch.setenv("WAN_ATTENTION_DUMP_DIR", str(tmp_path))
    n = 1100
    # keys close to their queries: each row attends mostly to itself, so the
    # 180 padded copies of the last key (weight ~1/n each) barely move it
    q32 = cpu_randn(1, n, 2, 128, seed=21).float()
    q = q32.to(torch.bfloat16).to(gpu)
    k = (q32 + 0.3 * cpu_randn(1, n, 2, 128, seed=22).float()).to(torch.bfloat16).to(gpu)
    v = cpu_randn(1, n, 2, 128, seed=23).to(gpu)
    wan_hook.set_quant_cfg(_cfg2())
    out = wan_hook.fake_or_sdpa_attention(q, k, v)
    rec = wan_hook.get_call_log()[0]
    ref = _softmax_attention_f64(q.cpu(), k.cpu(), v.cpu(), 128 ** -0.5)
    a, b = out.cpu().double().flatten(), ref.flatten()
    cos = (a @ b / (a.norm() * b.norm())).item()
    assert abs(rec["compare_sdpa"]["cosine"] - cos) < 1e-5
    assert abs(rec["compare_sdpa"]["max_abs"] - (a - b).abs().max().item()) < 1e-3
    assert cos > 0.99 and not rec["compare_sdpa"]["out_has_nan"]
    assert rec["compare_online_rowmax"]["cosine"] > 0.999
    assert not rec["compare_online_rowmax"]["ref_has_inf"]
    dump = torch.load(rec["dumped_qkv"], weights_only=True)
    assert torch.equal(dump["key"], k.cpu()) and dump["record"]["pad"] == 180
    assert torch.isfinite(out).all()
