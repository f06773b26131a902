"""CPU-side checks: the C-ABI library loads and exports every symbol
include/lbfq.h declares; host-side guards raise the reference's errors."""

import ctypes
import os
import re

import pytest
import torch

from conftest import PKG_DIR, REPO


def _declared_symbols():
    text = open(os.path.join(REPO, "include", "lbfq.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(lbfq_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    from low_bit_fake_quant import _lib
    path = _lib.LIB_PATH
    if not os.path.exists(path):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    syms = _declared_symbols()
    assert len(syms) >= 10
    for name in syms:
        assert hasattr(lib, name), name
    assert set(syms) == set(_lib.EXPORTED)


def test_struct_layouts_match_header():
    """ctypes structs mirror the C structs field by field (names, order)."""
    from low_bit_fake_quant import _lib
    text = open(os.path.join(REPO, "include", "lbfq.h")).read()
    for struct, cls in (("lbfq_rowtile_params", _lib.RowTileParams), ("lbfq_attn_params", _lib.AttnParams),
                        ("lbfq_sdpa_dequant_params", _lib.SdpaDequantParams), ("lbfq_sdpa_params", _lib.SdpaParams)):
        body = re.search(r"typedef struct \{((?:(?!typedef struct).)*?)\}\s*" + struct, text, flags=re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            parts = decl.split()
            rest = " ".join(parts[1:]) if parts[0] != "const" else " ".join(parts[2:])
            for n in rest.split(","):
                names.append(n.strip().lstrip("*").strip())
        assert names == [f[0] for f in cls._fields_], struct


def test_product_fails_loudly_without_gpu(monkeypatch):
    from low_bit_fake_quant import _lib
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(_lib.HipLibraryError):
        _lib.load()


def test_reference_guard_messages_on_cpu_tensors():
    from low_bit_fake_quant import (fake_quant_attention, fp8_block_quant, group_mean_q, kmeans_reorder_tokens,
                                    smooth_k)
    x = torch.zeros(1, 64, 2, 64)
    with pytest.raises(ValueError, match="must live on CUDA"):
        fp8_block_quant(x)
    with pytest.raises(ValueError, match="must be 4-D NHD"):
        fp8_block_quant(torch.zeros(64, 2, 64))
    with pytest.raises(ValueError, match="q/k/v must live on CUDA"):
        fake_quant_attention(x, x, x)
    with pytest.raises(ValueError, match="shapes must match"):
        fake_quant_attention(x, x, torch.zeros(1, 32, 2, 64))
    with pytest.raises(ValueError, match="k must be 4-D NHD on CUDA"):
        smooth_k(x)
    with pytest.raises(ValueError, match="q must be 4-D NHD on CUDA"):
        group_mean_q(x)
    with pytest.raises(ValueError, match="t must be 4-D NHD on CUDA"):
        kmeans_reorder_tokens(x, n_clusters=4)


def test_kernel_config_guards():
    from low_bit_fake_quant import QuantConfig
    from low_bit_fake_quant.attention_kernel import parse_blasst_fill, validate_kernel_config

    def v(**kw):
        validate_kernel_config(QuantConfig(**kw), s=1024, d=128, has_qm=kw.get("smoothing", "full") == "full",
                               has_v_alpha=kw.get("v_smooth_mode") == "per_block")

    v()
    with pytest.raises(ValueError, match="blasst_lambda must be in"):
        v(blasst_lambda=1.5)
    with pytest.raises(ValueError, match="unknown blasst_fill_mode"):
        v(blasst_lambda=0.1, blasst_fill="bogus")
    with pytest.raises(ValueError, match="blasst_fill_mode requires blasst_lambda"):
        v(blasst_fill="mean")
    with pytest.raises(ValueError, match=r"blasst UTA bins \(3\) must divide block_n"):
        v(blasst_lambda=0.1, blasst_fill="uta3")
    with pytest.raises(ValueError, match="p_mx_block_n .* currently must equal block_n"):
        v(v_quant="mxfp8", v_mxfp8_block_size=128)
    with pytest.raises(ValueError, match="q_smooth_block .* must be >= block_m"):
        v(q_smooth_block_size=32)
    with pytest.raises(ValueError, match="v_smooth_block .* must be >= block_n"):
        v(v_smooth_mode="per_block", v_smooth_block_size=32)
    with pytest.raises(ValueError, match="v_block_size .* must be >= block_n"):
        v(v_quant="fp8_block", v_fp8_block_size=32)
    # block_n = 128 runs; its guards follow the reference's
    v(p_requant_block_n=128, p_requant_block_m=128, q_smooth_block_size=256)
    with pytest.raises(ValueError, match="p_requant_block_n in"):
        v(p_requant_block_n=32, p_requant_block_m=32)
    with pytest.raises(ValueError, match=r"blasst UTA bins \(256\) must divide block_n \(128\)"):
        v(p_requant_block_n=128, blasst_lambda=0.1, blasst_fill="uta256")
    with pytest.raises(ValueError, match="v_block_size .* must be >= block_n"):
        v(p_requant_block_n=128, v_quant="fp8_block", v_fp8_block_size=64)
    with pytest.raises(ValueError, match="p_mx_block_n .* currently must equal block_n"):
        v(p_requant_block_n=128, v_quant="mxfp8", p_quant="mx", p_mx_block_n=64)
    assert parse_blasst_fill("mean_a1.5", alpha=1.0, uta_bins=16) == (2, 1.5, 1)
    assert parse_blasst_fill("uta16_a1.5", alpha=1.0, uta_bins=16) == (6, 1.5, 16)
    assert parse_blasst_fill("uta", alpha=2.0, uta_bins=8) == (6, 2.0, 8)
    assert parse_blasst_fill("thr_a0.25", alpha=1.0, uta_bins=16) == (5, 0.25, 1)


def test_wan_padding_and_inputs():
    from low_bit_fake_quant.wan import make_inputs, pad_length, pad_qkv, workloads
    ws = workloads()
    assert pad_length(32760, ws[1].cfg) == 32768
    assert pad_length(32760, ws[2].cfg) == 32768
    assert pad_length(75600, ws[4].cfg) == 75776
    w = ws[0]
    q, k, v = make_inputs(w, seed=0)
    q2, _, _ = make_inputs(w, seed=0)
    assert q.shape == (1, 1024, 2, 64) and q.dtype == torch.bfloat16 and torch.equal(q, q2)
    qs, ks, vs = (t[:, :1000] for t in (q, k, v))
    qp, kp, vp, n = pad_qkv(qs, ks, vs, ws[2].cfg)
    assert n == 1000 and qp.shape[1] == 1024
    assert torch.count_nonzero(qp[:, 1000:]) == 0
    assert torch.equal(kp[:, 1000:], ks[:, -1:].expand(1, 24, 2, 64))


def test_rowtile_rejects_hadamard_with_v_modes():
    """lbfq_rowtile applies the Hadamard rotation only with the Q/K quant modes
    (NONE, FP8_BLOCK, MX_QK); with a V mode it returns an error before any
    launch (host-side check, no GPU needed)."""
    from low_bit_fake_quant import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    lib.lbfq_rowtile.argtypes = [ctypes.POINTER(_lib.RowTileParams), ctypes.c_void_p]
    lib.lbfq_rowtile.restype = ctypes.c_int
    lib.lbfq_last_error.restype = ctypes.c_char_p
    for qm in (_lib.Q_CHANNEL, _lib.Q_MX_V, _lib.Q_CHANNEL_AMAX):
        p = _lib.RowTileParams()
        p.x = 0x1000; p.x_dtype = 2; p.B, p.S, p.H, p.D = 1, 256, 2, 128; p.R = 64
        p.hadamard = 1; p.had_scale = 1.0; p.quant_mode = qm
        p.codes = 0x2000; p.codes_layout = _lib.LAYOUT_BHDS; p.codes_spitch = 256
        p.scale = 0x3000; p.amax_table = 0x4000; p.mx_block = 32
        assert lib.lbfq_rowtile(ctypes.byref(p), None) != 0
        assert b"Hadamard" in lib.lbfq_last_error()


def test_sdpa_entry_points_reject_bad_arguments_without_a_gpu():
    """lbfq_sdpa_dequant / lbfq_sdpa_fwd validate their parameters before any
    HIP call: bad parameters return -1 with a message, with no device present.
    (No pointer is dereferenced on these paths; fake addresses are enough.)"""
    from low_bit_fake_quant import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = _lib.load(require_gpu=False)

    def err(rc):
        assert rc == -1
        return lib.lbfq_last_error().decode()

    assert "null params" in err(lib.lbfq_sdpa_fwd(None, None))
    assert "null params" in err(lib.lbfq_sdpa_dequant(None, None))
    fake = 0x1000
    p = _lib.SdpaParams(B=1, H=2, S=256, D=128, s_pitch=256, q=fake, k=fake, v_t=fake, sdpa_dtype=2,
                        sm_scale=0.125, out=fake, out_dtype=2)
    for field, value, msg in (("D", 96, "D must be 64 or 128"), ("s_pitch", 200, "multiple of 128"),
                              ("s_pitch", 128, "multiple of 128"), ("sdpa_dtype", 0, "bf16 or fp16"),
                              ("out_dtype", 7, "bad output dtype 7"), ("v_t", None, "missing tensor"),
                              ("qk_bias", fake, "bad qm groups")):
        saved = getattr(p, field)
        setattr(p, field, value)
        assert msg in err(lib.lbfq_sdpa_fwd(ctypes.byref(p), None)), field
        setattr(p, field, saved)
    d = _lib.SdpaDequantParams(B=1, H=2, S=256, D=64, s_pitch=256, q_codes=fake, k_codes=fake, v_codes_t=fake,
                               qk_mx=0, q_scale=fake, k_scale=fake, qk_block=64, v_kind=0, v_scale=fake,
                               sdpa_dtype=2, q_out=fake, k_out=fake, v_t_out=fake)
    for field, value, msg in (("D", 32, "D must be 64 or 128"), ("q_out", None, "missing output"),
                              ("sdpa_dtype", 0, "bf16 or fp16"), ("v_kind", 3, "bad v_kind 3"),
                              ("v_alpha", fake, "bad V smoothing block 0")):
        saved = getattr(d, field)
        setattr(d, field, value)
        assert msg in err(lib.lbfq_sdpa_dequant(ctypes.byref(d), None)), field
        setattr(d, field, saved)
