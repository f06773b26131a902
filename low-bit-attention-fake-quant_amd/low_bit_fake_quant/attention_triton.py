"""Kernel-level entry ``fake_quant_attention_triton`` (reference
``attention_triton.py:410-611``): the P-requant attention on already
fake-quantised BHSD tensors, as the reference's block studies call it
(``bench/eval_blasst_quant.py:179-209``) -- same arguments, guards, output
(B,H,S,D) in Q's dtype and optional BLASST statistics.

The reference runs bf16 dots on the dequantised values it is given; the
gfx950 kernel multiplies FP8 codes.  The inputs are therefore turned back
into codes:

* Q and K: fp8_block codes with FP32 scales.  The block is the first of
  ``block_m``, 128, 64, 32, 16 rows whose re-quantisation reproduces the
  input exactly (dequantised fp8_block values come back as the same codes);
  when none does (values that were never FP8), 16-row blocks are used and
  the result carries that FP8 rounding (a ``RequantWarning`` says so; the
  reference runs bf16 dots on those values).
* V (``v_bhsd_bf16``): the E4M3 codes of its values when they all are E4M3
  values (the "FP8-cast bf16" input of the reference), with ``v_scale_bhd``
  as the per-channel scale or ``v_block_scale_bsh`` as the fp8_block scale;
  otherwise (pre-dequantised bf16 with unit scales) per-channel FP8 codes
  whose scales multiply ``v_scale_bhd`` (with a ``RequantWarning``: the
  reference multiplies the bf16 values themselves).
* The qm correction (``qm_bhgd`` with ``k_smooth_bhsd``) becomes the
  kernel's per-group table; ``rowmax_est_bhs`` must be constant within each
  q_smooth_block group (the kernel holds one estimate per group, as the qm_k
  path produces it) and needs the qm correction.

Limits of the gfx950 kernel: block_n in {64, 128}; D in {64, 128}.
"""

from __future__ import annotations

import warnings

import torch

from ._ops import RowSource, qmk
from .attention import QuantizedOperands
from .attention_kernel import KERNEL_BLOCK_NS, launch_attention
from .config import QuantConfig
from .quant import fp8_block_dequant, fp8_block_quant, fp8_per_channel_quant

LOG2E = 1.4426950408889634


class RequantWarning(UserWarning):
    """The kernel-level entry re-quantised an input that was not FP8-valued:
    the gfx950 kernel multiplies FP8 codes, so the result carries an FP8
    rounding of that input which the reference (bf16 dots) does not apply."""


def _requant_qk(x_bhsd: torch.Tensor, block_m: int, P: int):
    """Head-major fp8_block codes (B,H,P,D) and scales (B,H,S/blk) of a BHSD
    tensor; returns (codes, scale, blk, exact)."""
    b, h, s, d = x_bhsd.shape
    nhd = x_bhsd.permute(0, 2, 1, 3).contiguous()
    cands = [block_m] + [c for c in (128, 64, 32, 16) if c != block_m]
    cands = [c for c in cands if c >= 16 and (c & (c - 1)) == 0 and s % c == 0]
    if not cands:
        raise ValueError(f"S={s} must be divisible by 16 to re-quantise Q/K into fp8_block codes")
    chosen = None
    for c in cands:
        codes, scale = fp8_block_quant(nhd, block_s=c)
        back = fp8_block_dequant(codes, scale, block_s=c, dtype=x_bhsd.dtype)
        if torch.equal(back, nhd):
            chosen = (codes, scale, c, True)
            break
    if chosen is None:
        c = min(cands)
        codes, scale = fp8_block_quant(nhd, block_s=c)
        chosen = (codes, scale, c, False)
    codes, scale, c, exact = chosen
    out = (torch.zeros if P > s else torch.empty)((b, h, P, d), dtype=torch.uint8, device=x_bhsd.device)
    out[:, :, :s] = codes.view(torch.uint8).permute(0, 2, 1, 3)
    return out, scale.permute(0, 2, 1).contiguous(), c, exact


def _v_codes(v_bhsd: torch.Tensor, v_scale_bhd: torch.Tensor, P: int, block_scale):
    """V^T codes (B,H,D,P) and the kernel's V scale tensor; returns
    (codes_t, scale, v_kind, exact) -- exact: V was E4M3-valued."""
    b, h, s, d = v_bhsd.shape
    codes_t = (torch.zeros if P > s else torch.empty)((b, h, d, P), dtype=torch.uint8, device=v_bhsd.device)
    f8 = v_bhsd.to(torch.float8_e4m3fn)
    if torch.equal(f8.to(v_bhsd.dtype), v_bhsd):
        codes_t[..., :s] = f8.view(torch.uint8).transpose(-1, -2)
        if block_scale is not None:
            return codes_t, block_scale, 1, True
        return codes_t, v_scale_bhd.float().contiguous(), 0, True
    if block_scale is not None:
        raise ValueError("v_block_scale_bsh needs V in raw FP8 value units (E4M3 values in bf16)")
    codes, scale = fp8_per_channel_quant(v_bhsd.permute(0, 2, 1, 3).contiguous())  # (B,S,H,D), (B,H,D)
    codes_t[..., :s] = codes.view(torch.uint8).permute(0, 2, 3, 1)
    return codes_t, (scale.float() * v_scale_bhd.float()).contiguous(), 0, False


def fake_quant_attention_triton(
    q_bhsd: torch.Tensor,
    k_bhsd: torch.Tensor,
    v_bhsd_bf16: torch.Tensor,
    v_scale_bhd: torch.Tensor,
    *,
    sm_scale: float,
    p_max_offset: int,
    block_m: int = 64,
    block_n: int = 64,
    v_alpha: torch.Tensor | None = None,
    v_smooth_block: int = 0,
    k_smooth_bhsd: torch.Tensor | None = None,
    qm_bhgd: torch.Tensor | None = None,
    q_smooth_block: int = 0,
    v_block_scale_bsh: torch.Tensor | None = None,
    v_block_size: int = 0,
    p_quant_mode: str = "elementwise",
    p_mx_block_n: int = 0,
    rowmax_est_bhs: torch.Tensor | None = None,
    rowmax_init_bhs: torch.Tensor | None = None,
    blasst_lambda: float | None = None,
    blasst_fill_mode: str = "zero",
    blasst_fill_alpha: float = 1.0,
    blasst_uta_bins: int = 16,
    return_blasst_stats: bool = False,
):
    """FA2-style fake-quant attention on BHSD tensors (attention_triton.py:410-611)."""
    ops, cfg, init = triton_operands(
        q_bhsd, k_bhsd, v_bhsd_bf16, v_scale_bhd, sm_scale=sm_scale, p_max_offset=p_max_offset, block_m=block_m,
        block_n=block_n, v_alpha=v_alpha, v_smooth_block=v_smooth_block, k_smooth_bhsd=k_smooth_bhsd,
        qm_bhgd=qm_bhgd, q_smooth_block=q_smooth_block, v_block_scale_bsh=v_block_scale_bsh,
        v_block_size=v_block_size, p_quant_mode=p_quant_mode, p_mx_block_n=p_mx_block_n,
        rowmax_est_bhs=rowmax_est_bhs, rowmax_init_bhs=rowmax_init_bhs, blasst_lambda=blasst_lambda,
        blasst_fill_mode=blasst_fill_mode, blasst_fill_alpha=blasst_fill_alpha, blasst_uta_bins=blasst_uta_bins)
    want_stats = return_blasst_stats and blasst_lambda is not None
    res = launch_attention(ops, cfg, float(sm_scale), q_bhsd.dtype, return_blasst_stats=want_stats,
                           rowmax_init=init)
    out, stats = res if want_stats else (res, None)
    o = out.permute(0, 2, 1, 3).contiguous()
    if return_blasst_stats:
        if stats is None:  # no BLASST: no decisions
            stats = torch.zeros(((ops.s + block_m - 1) // block_m, ops.b * ops.h, 2), dtype=torch.float32,
                                device=o.device)
        return o, stats
    return o


def triton_operands(q_bhsd, k_bhsd, v_bhsd_bf16, v_scale_bhd, *, sm_scale, p_max_offset, block_m=64, block_n=64,
                    v_alpha=None, v_smooth_block=0, k_smooth_bhsd=None, qm_bhgd=None, q_smooth_block=0,
                    v_block_scale_bsh=None, v_block_size=0, p_quant_mode="elementwise", p_mx_block_n=0,
                    rowmax_est_bhs=None, rowmax_init_bhs=None, blasst_lambda=None, blasst_fill_mode="zero",
                    blasst_fill_alpha=1.0, blasst_uta_bins=16):
    """The reference wrapper's guards, then the kernel's operands: returns
    (QuantizedOperands, QuantConfig, rowmax_init (B*H,S) log2 units or None)."""
    B, H, S, D = q_bhsd.shape
    assert k_bhsd.shape == (B, H, S, D)
    assert v_bhsd_bf16.shape == (B, H, S, D)
    assert v_scale_bhd.shape == (B, H, D)
    assert q_bhsd.dtype == torch.bfloat16
    assert k_bhsd.dtype == torch.bfloat16
    assert v_bhsd_bf16.dtype == torch.bfloat16
    assert v_scale_bhd.dtype == torch.float32
    if not q_bhsd.is_cuda:
        raise ValueError("q/k/v must live on CUDA")
    if block_n not in KERNEL_BLOCK_NS:
        raise ValueError(f"the gfx950 P-requant kernel runs block_n in {KERNEL_BLOCK_NS}; got {block_n}")
    if D not in (64, 128):
        raise ValueError(f"D must be 64 or 128; got {D}")
    if block_m <= 0:
        raise ValueError(f"block_m must be > 0; got {block_m}")

    has_v_alpha = v_alpha is not None
    if has_v_alpha:
        if v_smooth_block <= 0:
            raise ValueError("v_smooth_block must be > 0 when v_alpha is given")
        if v_smooth_block < block_n or v_smooth_block % block_n != 0:
            raise ValueError(f"v_smooth_block ({v_smooth_block}) must be >= block_n ({block_n}) "
                             "and an integer multiple of block_n")
        if S % v_smooth_block != 0:
            raise ValueError(f"S ({S}) must be divisible by v_smooth_block ({v_smooth_block})")
        assert v_alpha.shape == (B, S // v_smooth_block, H, D)
        assert v_alpha.dtype == torch.float32
    has_qm = qm_bhgd is not None
    if has_qm:
        if k_smooth_bhsd is None:
            raise ValueError("k_smooth_bhsd required with qm_bhgd")
        if q_smooth_block <= 0:
            raise ValueError("q_smooth_block must be > 0 with qm_bhgd")
        if q_smooth_block < block_m or q_smooth_block % block_m != 0:
            raise ValueError(f"q_smooth_block ({q_smooth_block}) must be >= block_m ({block_m}) "
                             "and an integer multiple of block_m")
        if S % q_smooth_block != 0:
            raise ValueError(f"S ({S}) must be divisible by q_smooth_block ({q_smooth_block})")
        assert k_smooth_bhsd.shape == (B, H, S, D)
        assert k_smooth_bhsd.dtype == torch.bfloat16
        assert qm_bhgd.shape == (B, S // q_smooth_block, H, D)
        assert qm_bhgd.dtype == torch.float32
    if rowmax_est_bhs is not None:
        assert rowmax_est_bhs.shape == (B, H, S)
        assert rowmax_est_bhs.dtype == torch.float32
    if rowmax_init_bhs is not None:
        if rowmax_est_bhs is not None:
            raise ValueError("rowmax_init_bhs and rowmax_est_bhs are mutually exclusive")
        assert rowmax_init_bhs.shape == (B, H, S)
        assert rowmax_init_bhs.dtype == torch.float32
    v_kind_block = v_block_scale_bsh is not None
    if v_kind_block:
        assert v_block_scale_bsh.dtype == torch.float32
        if v_block_size <= 0:
            raise ValueError("v_block_size must be > 0 when v_block_scale_bsh is given")
        if v_block_size < block_n or v_block_size % block_n != 0:
            raise ValueError(f"v_block_size ({v_block_size}) must be >= block_n ({block_n}) "
                             "and an integer multiple of block_n")
        if S % v_block_size != 0:
            raise ValueError(f"S ({S}) must be divisible by v_block_size ({v_block_size})")
        assert v_block_scale_bsh.shape == (B, S // v_block_size, H)
    if p_quant_mode == "mx":
        if p_mx_block_n <= 0:
            raise ValueError("p_mx_block_n must be > 0 when p_quant_mode='mx'")
        if p_mx_block_n != block_n:
            raise ValueError(f"p_mx_block_n ({p_mx_block_n}) currently must equal block_n ({block_n}); "
                             "sub-block scaling within a K block is not implemented")
    elif p_quant_mode not in ("elementwise", "dynamic"):
        raise ValueError(f"unknown p_quant_mode: {p_quant_mode!r}")
    if blasst_lambda is not None:
        if not (0.0 < float(blasst_lambda) < 1.0):
            raise ValueError(f"blasst_lambda must be in (0, 1); got {blasst_lambda}")
    elif blasst_fill_mode not in ("zero", None):
        raise ValueError("blasst_fill_mode requires blasst_lambda")
    if rowmax_est_bhs is not None and not has_qm:
        raise NotImplementedError("the gfx950 kernel takes a fixed row-max estimate together with the qm "
                                  "correction (qm_bhgd / k_smooth_bhsd)")

    P = (S + 127) // 128 * 128
    q_codes, q_scale, qblk, q_exact = _requant_qk(q_bhsd, block_m, P)
    k_codes, k_scale, kblk, k_exact = _requant_qk(k_bhsd, block_m, P)
    if kblk != qblk:  # one block size for both (the kernel reads one fp8_block size)
        blk = min(qblk, kblk)
        q_codes, q_scale, _, q_exact = _requant_qk(q_bhsd, blk, P)
        k_codes, k_scale, _, k_exact = _requant_qk(k_bhsd, blk, P)
        qblk = blk
    if not (q_exact and k_exact):
        warnings.warn(f"Q/K are not fp8_block-dequantised values; re-quantised to {qblk}-row FP8 blocks "
                      "(the reference runs bf16 dots on them)", RequantWarning, stacklevel=3)
    bscale = v_block_scale_bsh.permute(0, 2, 1).contiguous() if v_kind_block else None
    v_codes_t, v_scale, v_kind, v_exact = _v_codes(v_bhsd_bf16, v_scale_bhd, P, bscale)
    if not v_exact:
        warnings.warn("V is not E4M3-valued; re-quantised to per-channel FP8 codes (the reference multiplies "
                      "the bf16 values)", RequantWarning, stacklevel=3)
    if has_v_alpha and v_kind == 0 and not bool((torch.isfinite(v_scale) & (v_scale > 0)).all()):
        # the kernel holds the V-smoothing correction in the accumulator's
        # units (alpha / v_scale) so the epilogue's per-channel multiply
        # restores it; a zero or non-finite channel scale has no such form
        raise ValueError("v_scale_bhd must be finite and > 0 in every channel when v_alpha is given")
    bias = rowmax = None
    if has_qm:
        ks_nhd = k_smooth_bhsd.permute(0, 2, 1, 3).contiguous()
        bias, _ = qmk(qm_bhgd.contiguous(), RowSource(ks_nhd), float(sm_scale) * LOG2E, s_pitch=P,
                      want_rowmax=False)
        if rowmax_est_bhs is not None:
            g = rowmax_est_bhs.view(B, H, S // q_smooth_block, q_smooth_block)
            if not torch.equal(g, g[..., :1].expand_as(g)):
                raise NotImplementedError("the gfx950 kernel holds one row-max estimate per q_smooth_block "
                                          "group; rowmax_est_bhs varies within a group")
            rowmax = (g[..., 0] * LOG2E).contiguous()
    va = None
    if has_v_alpha:
        va = v_alpha.permute(0, 2, 1, 3).contiguous()
        if v_kind == 0:
            va = va / v_scale[:, :, None, :]
    ops = QuantizedOperands(b=B, s=S, h=H, d=D, P=P, q_codes=q_codes, q_scale=q_scale, k_codes=k_codes,
                            k_scale=k_scale, v_codes_t=v_codes_t, v_scale=v_scale, v_kind=v_kind,
                            v_block=v_block_size if v_kind_block else 0, bias=bias, rowmax=rowmax, v_alpha=va,
                            out_row_map=None)
    cfg = QuantConfig(qk_quant="fp8_block", fp8_block_size=qblk, v_quant="fp8_block" if v_kind_block else "fp8_channel",
                      v_fp8_block_size=v_block_size if v_kind_block else 128, smoothing="full" if has_qm else "off",
                      q_smooth_block_size=q_smooth_block if has_qm else 256, q_kmeans_k=None, p_requant=True,
                      p_quant=p_quant_mode, p_max_offset=int(p_max_offset), p_mx_block_n=p_mx_block_n,
                      rowmax_mode="qm_k" if rowmax is not None else "online", p_requant_block_m=block_m,
                      p_requant_block_n=block_n, v_smooth_mode="per_block" if has_v_alpha else "off",
                      v_smooth_block_size=v_smooth_block if has_v_alpha else 64, blasst_lambda=blasst_lambda,
                      blasst_fill=blasst_fill_mode, blasst_fill_alpha=blasst_fill_alpha,
                      blasst_uta_bins=blasst_uta_bins)
    init = None
    if rowmax_init_bhs is not None:
        init = (rowmax_init_bhs.float() * LOG2E).reshape(B * H, S).contiguous()
    return ops, cfg, init


__all__ = ["fake_quant_attention_triton", "RequantWarning"]
