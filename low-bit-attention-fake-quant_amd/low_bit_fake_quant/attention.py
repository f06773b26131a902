"""``fake_quant_attention`` on MI355X: the drop-in entry point.

Public API and error messages follow the reference's ``attention.py``
(FakeQuantArtifacts :77-86, PreprocessCache :647-670, prepare_for_attention
:673-703, fake_quant_attention :706-806, reference_attention :809-825).

Execution differs from the reference in how the work is laid out:

* The preprocess (``attention.py:166-239``: Q k-means, K smoothing, Q group
  mean, V k-means with K co-permutation, V per-block smoothing) is kept
  *lazy*: each operand is described by a source tensor, a row gather and a
  mean table, and the quantiser pass applies gather -> subtract -> round ->
  (Hadamard) -> quantise in one read of the source.  ``prepare_for_attention``
  materialises the same work tensors as the reference for callers that cache
  them.
* P-requant path (``attention.py:505-639``): Q/K are quantised straight into
  head-major FP8 codes, V into transposed FP8 codes, the qm correction and
  the qm_k row-max estimate come from one qm.K_s pass, and one FP8-MFMA kernel
  computes attention, writing rows directly to their original (pre-k-means)
  positions of the NHD output.
* SDPA path (``attention.py:245-321``): the same prepass quantisers, a
  dequantisation into the SDPA dtype (V transposed, V block means added), and
  one bf16/fp16-MFMA flash-attention kernel with P not quantised, writing rows
  directly to their original positions.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._ops import RowSource, channel_amax, colsum_mean, column_mean, hadamard_scale, qmk, round_up, rowtile
from .attention_kernel import launch_attention, v_tile_colsum, validate_kernel_config
from .config import QuantConfig
from .hadamard import apply_qk_hadamard, qk_signs_device
from .kmeans import KMeansReorderResult, kmeans_labels, make_result
from .quant import (
    fp8_block_dequant,
    fp8_block_quant,
    fp8_per_channel_dequant,
    fp8_per_channel_quant,
    mxfp8_qk_dequant,
    mxfp8_qk_quant,
    mxfp8_v_dequant,
    mxfp8_v_quant,
)

LOG2E = 1.4426950408889634


@dataclass
class FakeQuantArtifacts:
    """Side data emitted by :func:`fake_quant_attention` for debugging."""

    qm: Optional[torch.Tensor] = None
    k_mean: Optional[torch.Tensor] = None
    kmeans: Optional[KMeansReorderResult] = None
    q_eff_dtype: Optional[torch.dtype] = None
    p_requant: bool = False
    qk_hadamard: bool = False


@dataclass
class PreprocessCache:
    """Cached output of :func:`prepare_for_attention` (reference attention.py:647-670)."""

    q_work: torch.Tensor
    k_work: torch.Tensor
    v_work: torch.Tensor
    qm: Optional[torch.Tensor]
    v_alpha: Optional[torch.Tensor]
    q_kmeans: Optional[KMeansReorderResult]
    v_kmeans: Optional[KMeansReorderResult]
    smoothing: str
    q_kmeans_k: Optional[int]
    q_smooth_block_size: int
    v_smooth_mode: str
    v_smooth_block_size: int
    v_kmeans_k: Optional[int]


@dataclass
class _Prep:
    """Lazy preprocess state: each operand as a RowSource."""

    q: RowSource
    k: RowSource
    v: RowSource
    qm: Optional[torch.Tensor]
    v_alpha: Optional[torch.Tensor]
    k_mean: Optional[torch.Tensor]
    q_km: Optional[tuple]          # (labels, order, inverse) int32
    v_km: Optional[tuple]
    q_km_result: Optional[KMeansReorderResult] = None

    def work(self, which: str) -> torch.Tensor:
        src = getattr(self, which)
        if src.gather is None and src.sub_mode == _lib.SUB_NONE:
            return src.x
        out = torch.empty_like(src.x)
        rowtile(src, R=64, smoothed=out)
        return out

    def q_order_i32(self) -> Optional[torch.Tensor]:
        if self.q_km is not None:
            return self.q_km[1]
        if self.q_km_result is not None:
            r = self.q_km_result
            return r.order_i32 if r.order_i32 is not None else r.order.to(torch.int32).contiguous()
        return None

    def q_inverse_i32(self) -> Optional[torch.Tensor]:
        if self.q_km is not None:
            return self.q_km[2]
        if self.q_km_result is not None:
            r = self.q_km_result
            return r.inverse_i32 if r.inverse_i32 is not None else r.inverse_order.to(torch.int32).contiguous()
        return None


def _lazy_preprocess(q, k, v, cfg: QuantConfig) -> _Prep:
    """Reference order (attention.py:180-189): Q kmeans -> K smooth -> Q smooth ->
    V kmeans (+ K co-permute) -> V smooth, without materialising anything."""
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    b, s, h, d = q.shape
    q_src, k_src, v_src = RowSource(q), RowSource(k), RowSource(v)
    q_km = v_km = None
    if cfg.q_kmeans_k is not None:
        q_km = kmeans_labels(q, n_clusters=cfg.q_kmeans_k, max_iters=cfg.q_kmeans_iters, seed=cfg.q_kmeans_seed)
        q_src = RowSource(q, gather=q_km[1])
    qm = k_mean = None
    if cfg.smoothing == "off":
        pass
    elif cfg.smoothing in ("k_only", "full"):
        if d not in (64, 128):
            raise ValueError(f"D must be 64 or 128; got {d}")
        k_mean = column_mean(k)
        k_src = RowSource(k, sub_mode=_lib.SUB_COLVEC, sub=k_mean)
        if cfg.smoothing == "full":
            block_q = cfg.q_smooth_block_size
            if s % block_q != 0:
                raise ValueError(f"S={s} must be divisible by block_q={block_q}")
            qm = colsum_mean(q, block_q, gather=q_src.gather)
            q_src = RowSource(q, gather=q_src.gather, sub_mode=_lib.SUB_BLOCKVEC, sub=qm, sub_block=block_q)
    else:
        raise ValueError(f"unsupported smoothing: {cfg.smoothing!r}")
    if cfg.v_kmeans_k is not None:
        v_km = kmeans_labels(v, n_clusters=cfg.v_kmeans_k, max_iters=cfg.v_kmeans_iters, seed=cfg.v_kmeans_seed)
        v_src = RowSource(v, gather=v_km[1])
        k_src = RowSource(k, gather=v_km[1], sub_mode=k_src.sub_mode, sub=k_src.sub)
    v_alpha = None
    if cfg.v_smooth_mode == "off":
        pass
    elif cfg.v_smooth_mode == "per_block":
        vsb = cfg.v_smooth_block_size
        if s % vsb != 0:
            raise ValueError(f"S={s} must be divisible by block_s={vsb}")
        if d not in (64, 128):
            raise ValueError(f"D must be 64 or 128; got {d}")
        v_alpha = colsum_mean(v, vsb, gather=v_src.gather)
        v_src = RowSource(v, gather=v_src.gather, sub_mode=_lib.SUB_BLOCKVEC, sub=v_alpha, sub_block=vsb)
    else:
        raise ValueError(f"unsupported v_smooth_mode: {cfg.v_smooth_mode!r}")
    return _Prep(q=q_src, k=k_src, v=v_src, qm=qm, v_alpha=v_alpha, k_mean=k_mean, q_km=q_km, v_km=v_km)


def _prep_from_cache(c: PreprocessCache) -> _Prep:
    return _Prep(q=RowSource(c.q_work.contiguous()), k=RowSource(c.k_work.contiguous()),
                 v=RowSource(c.v_work.contiguous()), qm=c.qm, v_alpha=c.v_alpha, k_mean=None, q_km=None,
                 v_km=None, q_km_result=c.q_kmeans)


def _kmeans_result(src_tensor, km) -> Optional[KMeansReorderResult]:
    if km is None:
        return None
    labels, order, inverse = km
    return make_result(src_tensor, labels, order, inverse)


# ---------------------------------------------------------------------------
# Path B: FP8-MFMA P-requant attention
# ---------------------------------------------------------------------------


def _quant_qk_codes(src: RowSource, cfg: QuantConfig, P: int, *, signs):
    """Quantise one of Q/K into head-major codes (B,H,P,D) and the kernel's scales:
    fp8_block -> (B,H,S/block) fp32; mxfp8 -> (B,H,P,D/32) E8M0 bytes."""
    b, s, h, d = src.shape
    dev = src.x.device
    codes = (torch.zeros if P > s else torch.empty)((b, h, P, d), dtype=torch.uint8, device=dev)
    hs = hadamard_scale(d)
    if cfg.qk_quant == "fp8_block":
        blk = cfg.fp8_block_size
        if s % blk != 0:
            raise ValueError(f"S={s} must be divisible by block_s={blk}")
        nb = s // blk
        scale = torch.empty((b, h, nb), dtype=torch.float32, device=dev)
        rowtile(src, R=blk, hadamard=cfg.qk_hadamard, signs=signs, had_scale=hs, quant_mode=_lib.Q_FP8_BLOCK,
                codes=codes, codes_layout=_lib.LAYOUT_BHSD, codes_spitch=P, scale=scale,
                scale_strides=(h * nb, 1, nb, 0))
    elif cfg.qk_quant == "mxfp8":
        bd = cfg.mxfp8_block_size
        if d % bd != 0:
            raise ValueError(f"D={d} must be divisible by block_d={bd}")
        nb = d // bd
        # padding rows keep E8M0 0 (2^-127): finite, and their codes are zero
        scale = torch.zeros((b, h, P, nb), dtype=torch.uint8, device=dev)
        rowtile(src, R=64, hadamard=cfg.qk_hadamard, signs=signs, had_scale=hs, quant_mode=_lib.Q_MX_QK,
                codes=codes, codes_layout=_lib.LAYOUT_BHSD, codes_spitch=P, scale=scale,
                scale_strides=(h * P * nb, nb, P * nb, 1), mx_block=bd, scale_e8m0=True)
    else:
        raise ValueError(f"unsupported qk_quant: {cfg.qk_quant!r}")
    return codes, scale


def _quant_v_codes(src: RowSource, cfg: QuantConfig, P: int):
    """Quantise V into transposed codes (B,H,D,P) and the kernel's scales:
    channel (B,H,D) fp32, fp8_block (B,H,S/vb) fp32, mxfp8 (B,H,S/vb,D) E8M0.
    Returns (codes_t, scale, v_kind, v_block)."""
    b, s, h, d = src.shape
    dev = src.x.device
    codes = (torch.zeros if P > s else torch.empty)((b, h, d, P), dtype=torch.uint8, device=dev)
    if cfg.v_quant == "fp8_channel":
        table = channel_amax(src)
        scale = torch.empty((b, h, d), dtype=torch.float32, device=dev)
        rowtile(src, R=64, quant_mode=_lib.Q_CHANNEL, codes=codes, codes_layout=_lib.LAYOUT_BHDS, codes_spitch=P,
                scale=scale, scale_strides=(scale.stride(0), 0, scale.stride(1), scale.stride(2)), amax_table=table)
        return codes, scale, 0, 0
    if cfg.v_quant == "fp8_block":
        vb = cfg.v_fp8_block_size
        if s % vb != 0:
            raise ValueError(f"S={s} must be divisible by block_s={vb}")
        nb = s // vb
        scale = torch.empty((b, h, nb), dtype=torch.float32, device=dev)
        rowtile(src, R=vb, quant_mode=_lib.Q_FP8_BLOCK, codes=codes, codes_layout=_lib.LAYOUT_BHDS, codes_spitch=P,
                scale=scale, scale_strides=(h * nb, 1, nb, 0))
        return codes, scale, 1, vb
    if cfg.v_quant == "mxfp8":
        vb = cfg.v_mxfp8_block_size
        if s % vb != 0:
            raise ValueError(f"S={s} must be divisible by block_s={vb}")
        nb = s // vb
        scale = torch.empty((b, h, nb, d), dtype=torch.uint8, device=dev)
        rowtile(src, R=vb, quant_mode=_lib.Q_MX_V, codes=codes, codes_layout=_lib.LAYOUT_BHDS, codes_spitch=P,
                scale=scale, scale_strides=(h * nb * d, d, nb * d, 1), scale_e8m0=True)
        return codes, scale, 2, vb
    raise ValueError(f"unsupported v_quant: {cfg.v_quant!r}")


@dataclass
class QuantizedOperands:
    """Everything the attention kernel reads, in its HBM layouts (head-major,
    S padded to the pitch P with zero codes)."""

    b: int
    s: int
    h: int
    d: int
    P: int
    q_codes: torch.Tensor                 # (B,H,P,D) E4M3
    q_scale: torch.Tensor                 # fp8_block (B,H,S/blk) fp32 | mx (B,H,P,D/32) E8M0
    k_codes: torch.Tensor                 # (B,H,P,D) E4M3
    k_scale: torch.Tensor
    v_codes_t: torch.Tensor               # (B,H,D,P) E4M3
    v_scale: torch.Tensor                 # channel (B,H,D) | block (B,H,S/vb) | mx (B,H,S/vb,D) E8M0
    v_kind: int
    v_block: int
    bias: Optional[torch.Tensor]          # (B,H,G,P) qm.K_s * sm_scale * log2(e)
    rowmax: Optional[torch.Tensor]        # (B,H,G) max_n bias (log2 units)
    v_alpha: Optional[torch.Tensor]       # (B,H,S/vsb,D) fp32 block means (/ channel V scale)
    out_row_map: Optional[torch.Tensor]   # (B*H,S) int32
    v_colsum: Optional[torch.Tensor] = None  # (B*H,P/64,D) fp32 V tile column sums (BLASST PV skip)


def quantize_operands(prep: _Prep, cfg: QuantConfig, sm_scale: float) -> QuantizedOperands:
    """The prepass: codes, scales, qm correction and row-max estimate."""
    b, s, h, d = prep.q.shape
    has_qm = prep.qm is not None
    validate_kernel_config(cfg, s=s, d=d, has_qm=has_qm, has_v_alpha=prep.v_alpha is not None)
    # the pitch: a multiple of 256 (at most 255 zero rows), which the attention
    # kernel's eight-wave (256-query) workgroups require
    P = round_up(s, 256)
    signs = None
    if cfg.qk_hadamard and cfg.qk_hadamard_random_sign:
        signs = qk_signs_device(h, d, cfg.qk_hadamard_seed, prep.q.x.device)
    if cfg.rowmax_mode == "qm_k":
        if not has_qm:
            raise ValueError("rowmax_mode='qm_k' requires smoothing='full' so qm exists")
    elif cfg.rowmax_mode != "online":
        raise ValueError(f"unsupported rowmax_mode: {cfg.rowmax_mode!r}")
    q_codes, q_scale = _quant_qk_codes(prep.q, cfg, P, signs=signs)
    # with the qm correction, K_s is quantised inside the qm.K_s pass when it can be
    fuse_k = has_qm and _k_quant_fusable(prep.k, cfg, P, prep.qm.shape[1])
    if fuse_k:
        blk = cfg.fp8_block_size
        k_codes = (torch.zeros if P > s else torch.empty)((b, h, P, d), dtype=torch.uint8, device=prep.k.x.device)
        k_scale = torch.empty((b, h, s // blk), dtype=torch.float32, device=prep.k.x.device)
    else:
        k_codes, k_scale = _quant_qk_codes(prep.k, cfg, P, signs=signs)
    v_codes, v_scale, v_kind, v_block = _quant_v_codes(prep.v, cfg, P)
    bias = rowmax = None
    if has_qm:
        # scores are handled in log2 units by the kernel
        # K_s = K - mean is formed inside the qm.K_s kernel (never stored)
        bias, rowmax = qmk(prep.qm, prep.k, sm_scale * LOG2E, s_pitch=P, want_rowmax=cfg.rowmax_mode == "qm_k",
                           k_quant=(k_codes, k_scale, cfg.fp8_block_size) if fuse_k else None)
    v_alpha = None
    if prep.v_alpha is not None:
        v_alpha = prep.v_alpha.permute(0, 2, 1, 3).contiguous()
        if v_kind == 0:
            # the kernel adds the V-smoothing correction into its accumulator,
            # which the per-channel V scales multiply at the end
            v_alpha = v_alpha / v_scale[:, :, None, :]
    v_colsum = None
    if cfg.blasst_lambda is not None and v_alpha is None and cfg.p_requant_block_n == 64:
        # lets the kernel apply a tile that all rows of a wave skip as fill x column sums
        v_colsum = v_tile_colsum(v_codes, v_scale, v_kind, v_block, s)
    return QuantizedOperands(b=b, s=s, h=h, d=d, P=P, q_codes=q_codes, q_scale=q_scale, k_codes=k_codes,
                             k_scale=k_scale, v_codes_t=v_codes, v_scale=v_scale, v_kind=v_kind, v_block=v_block,
                             bias=bias, rowmax=rowmax, v_alpha=v_alpha, out_row_map=prep.q_order_i32(),
                             v_colsum=v_colsum)


def _p_requant_hip(prep: _Prep, cfg: QuantConfig, sm_scale: float, out_dtype: torch.dtype,
                   return_blasst_stats: bool = False):
    ops = quantize_operands(prep, cfg, sm_scale)
    return launch_attention(ops, cfg, sm_scale, out_dtype, return_blasst_stats=return_blasst_stats)


# ---------------------------------------------------------------------------
# Path A: dequant Q/K/V -> attention with P not quantised (reference attention.py:245-321)
# ---------------------------------------------------------------------------


def _k_quant_fusable(k: RowSource, cfg: QuantConfig, P: int, groups: int) -> bool:
    """Whether lbfq_qmk_kquant can quantise K_s in the qm.K_s pass: bf16 K,
    fp8_block of 16/32/64 keys, no Hadamard, a table under 4 GiB per head."""
    s = k.shape[1]
    return (cfg.qk_quant == "fp8_block" and not cfg.qk_hadamard and k.x.dtype == torch.bfloat16
            and cfg.fp8_block_size in (16, 32, 64) and s % cfg.fp8_block_size == 0
            and k.sub_mode in (_lib.SUB_NONE, _lib.SUB_COLVEC) and groups * P * 4 < (1 << 32))


# Quantise / dequantise helpers of the reference's path A (attention.py:89-160),
# kept under the same names because callers and the reference's own tests use
# them (tests/test_qk_hadamard.py imports the Q/K ones): NHD tensors through the
# HIP quantisers of quant.py.  The native path A above does not go through them.


def _qk_inputs_for_quant(q_work, k_work, cfg):
    if not cfg.qk_hadamard:
        return q_work, k_work
    return apply_qk_hadamard(q_work, k_work, random_sign=cfg.qk_hadamard_random_sign, seed=cfg.qk_hadamard_seed)


def _quant_qk(t, cfg):
    if cfg.qk_quant == "fp8_block":
        c, sc = fp8_block_quant(t, block_s=cfg.fp8_block_size)
        return c, sc, {"kind": "fp8_block", "block_s": cfg.fp8_block_size}
    if cfg.qk_quant == "mxfp8":
        c, sc = mxfp8_qk_quant(t, block_d=cfg.mxfp8_block_size)
        return c, sc, {"kind": "mxfp8", "block_d": cfg.mxfp8_block_size}
    raise ValueError(f"unsupported qk_quant: {cfg.qk_quant!r}")


def _dequant_qk(fp8, scale, meta, dtype):
    if meta["kind"] == "fp8_block":
        return fp8_block_dequant(fp8, scale, block_s=meta["block_s"], dtype=dtype)
    if meta["kind"] == "mxfp8":
        return mxfp8_qk_dequant(fp8, scale, block_d=meta["block_d"], dtype=dtype)
    raise ValueError(f"bad meta: {meta!r}")


def _quant_v(t, cfg):
    if cfg.v_quant == "fp8_channel":
        c, sc = fp8_per_channel_quant(t)
        return c, sc, {"kind": "fp8_channel"}
    if cfg.v_quant == "fp8_block":
        c, sc = fp8_block_quant(t, block_s=cfg.v_fp8_block_size)
        return c, sc, {"kind": "fp8_block", "block_s": cfg.v_fp8_block_size}
    if cfg.v_quant == "mxfp8":
        c, sc = mxfp8_v_quant(t, block_s=cfg.v_mxfp8_block_size)
        return c, sc, {"kind": "mxfp8", "block_s": cfg.v_mxfp8_block_size}
    raise ValueError(f"unsupported v_quant: {cfg.v_quant!r}")


def _dequant_v(fp8, scale, meta, dtype):
    if meta["kind"] == "fp8_channel":
        return fp8_per_channel_dequant(fp8, scale, dtype=dtype)
    if meta["kind"] == "fp8_block":
        return fp8_block_dequant(fp8, scale, block_s=meta["block_s"], dtype=dtype)
    if meta["kind"] == "mxfp8":
        return mxfp8_v_dequant(fp8, scale, block_s=meta["block_s"], dtype=dtype)
    raise ValueError(f"bad meta: {meta!r}")


@dataclass
class SdpaOperands:
    """Path A's operands in the SDPA dtype, head-major, S padded to the pitch P
    with zeros, plus the qm correction table."""

    b: int
    s: int
    h: int
    d: int
    P: int
    q: torch.Tensor                       # (B,H,P,D) sdpa dtype
    k: torch.Tensor                       # (B,H,P,D)
    v_t: torch.Tensor                     # (B,H,D,P), V block means added
    bias: Optional[torch.Tensor]          # (B,H,G,P) qm.K_s * sm_scale * log2(e)
    q_group: int
    out_row_map: Optional[torch.Tensor]   # (B*H,S) int32


def sdpa_operands(prep: _Prep, cfg: QuantConfig, sm_scale: float, sdpa_dtype: torch.dtype) -> SdpaOperands:
    """Quantise Q/K/V with the reference's quantisers (attention.py:271-273: the
    same codes as the P-requant path's prepass), dequantise them into the SDPA
    dtype and add the V block means (attention.py:274-286), and form the qm
    correction of the Q-smoothing branch (attention.py:311-312)."""
    b, s, h, d = prep.q.shape
    dev = prep.q.x.device
    P = round_up(s, 128)
    signs = None
    if cfg.qk_hadamard and cfg.qk_hadamard_random_sign:
        signs = qk_signs_device(h, d, cfg.qk_hadamard_seed, dev)
    q_codes, q_scale = _quant_qk_codes(prep.q, cfg, P, signs=signs)
    k_codes, k_scale = _quant_qk_codes(prep.k, cfg, P, signs=signs)
    v_codes, v_scale, v_kind, v_block = _quant_v_codes(prep.v, cfg, P)
    v_alpha = None
    if prep.v_alpha is not None:
        if s % cfg.v_smooth_block_size != 0:
            raise ValueError(f"S={s} not divisible by v_smooth_block_size={cfg.v_smooth_block_size}")
        v_alpha = prep.v_alpha.permute(0, 2, 1, 3).float().contiguous()
    q_deq = torch.empty((b, h, P, d), dtype=sdpa_dtype, device=dev)
    k_deq = torch.empty_like(q_deq)
    v_t = torch.empty((b, h, d, P), dtype=sdpa_dtype, device=dev)
    mx = cfg.qk_quant == "mxfp8"
    p = _lib.SdpaDequantParams(
        B=b, H=h, S=s, D=d, s_pitch=P, q_codes=q_codes.data_ptr(), k_codes=k_codes.data_ptr(),
        v_codes_t=v_codes.data_ptr(), qk_mx=int(mx), q_scale=q_scale.data_ptr(), k_scale=k_scale.data_ptr(),
        qk_block=cfg.mxfp8_block_size if mx else cfg.fp8_block_size, v_kind=v_kind, v_scale=v_scale.data_ptr(),
        v_block=v_block, v_alpha=_lib.ptr(v_alpha), v_smooth_block=cfg.v_smooth_block_size if v_alpha is not None
        else 0, sdpa_dtype=_lib.DTYPE_CODE[sdpa_dtype], q_out=q_deq.data_ptr(), k_out=k_deq.data_ptr(),
        v_t_out=v_t.data_ptr())
    _lib.check(_lib.load().lbfq_sdpa_dequant(p, _lib.stream_handle(dev)), "lbfq_sdpa_dequant")
    bias = None
    if prep.qm is not None:
        bias, _ = qmk(prep.qm, prep.k, sm_scale * LOG2E, s_pitch=P, want_rowmax=False)
    return SdpaOperands(b=b, s=s, h=h, d=d, P=P, q=q_deq, k=k_deq, v_t=v_t, bias=bias,
                        q_group=cfg.q_smooth_block_size, out_row_map=prep.q_order_i32())


def launch_sdpa(ops: SdpaOperands, sm_scale: float, out_dtype: torch.dtype) -> torch.Tensor:
    """The attention of path A (attention.py:288-319) on the dequantised operands:
    NHD output in ``out_dtype`` (values rounded to the SDPA dtype), rows in
    their original (pre-k-means) positions."""
    dev = ops.q.device
    out = torch.empty((ops.b, ops.s, ops.h, ops.d), dtype=out_dtype, device=dev)
    p = _lib.SdpaParams(
        B=ops.b, H=ops.h, S=ops.s, D=ops.d, s_pitch=ops.P, q=ops.q.data_ptr(), k=ops.k.data_ptr(),
        v_t=ops.v_t.data_ptr(), sdpa_dtype=_lib.DTYPE_CODE[ops.q.dtype], sm_scale=float(sm_scale),
        qk_bias=_lib.ptr(ops.bias), groups=ops.bias.shape[2] if ops.bias is not None else 0,
        q_group=ops.q_group if ops.bias is not None else 0, out=out.data_ptr(), out_dtype=_lib.DTYPE_CODE[out_dtype],
        out_row_map=_lib.ptr(ops.out_row_map))
    _lib.check(_lib.load().lbfq_sdpa_fwd(p, _lib.stream_handle(dev)), "lbfq_sdpa_fwd")
    return out


def _sdpa_hip(prep: _Prep, cfg: QuantConfig, sm_scale: float, out_dtype: torch.dtype,
              sdpa_dtype: torch.dtype) -> torch.Tensor:
    return launch_sdpa(sdpa_operands(prep, cfg, sm_scale, sdpa_dtype), sm_scale, out_dtype)


def _attention_fp32(qb, kb, vb, sm_scale, *, chunk=512):
    """softmax(q k^T * scale) v over BHSD tensors in fp32 with contiguous
    operands, chunked over queries (bounded memory)."""
    B, H, S, D = qb.shape
    kT = kb.float().transpose(-2, -1).contiguous()
    vf = vb.float().contiguous()
    out = torch.empty((B, H, S, D), dtype=torch.float32, device=qb.device)
    for m0 in range(0, S, chunk):
        m1 = min(m0 + chunk, S)
        scores = torch.matmul(qb[:, :, m0:m1].float().contiguous(), kT) * sm_scale
        out[:, :, m0:m1] = torch.matmul(torch.softmax(scores, dim=-1), vf)
    return out


# ---------------------------------------------------------------------------
# Public entry points
# ---------------------------------------------------------------------------


def prepare_for_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cfg: QuantConfig) -> PreprocessCache:
    """Run k-means + Q/K smoothing + V smoothing without quantisation and
    materialise the work tensors (reusable across quant configurations)."""
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q/k/v shapes must match")
    if q.ndim != 4 or not q.is_cuda:
        raise ValueError("q/k/v must be 4-D NHD on CUDA")
    prep = _lazy_preprocess(q, k, v, cfg)
    return PreprocessCache(
        q_work=prep.work("q"), k_work=prep.work("k"), v_work=prep.work("v"), qm=prep.qm, v_alpha=prep.v_alpha,
        q_kmeans=_kmeans_result(q.contiguous(), prep.q_km), v_kmeans=_kmeans_result(v.contiguous(), prep.v_km),
        smoothing=cfg.smoothing, q_kmeans_k=cfg.q_kmeans_k, q_smooth_block_size=cfg.q_smooth_block_size,
        v_smooth_mode=cfg.v_smooth_mode, v_smooth_block_size=cfg.v_smooth_block_size, v_kmeans_k=cfg.v_kmeans_k)


def fake_quant_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cfg: Optional[QuantConfig] = None,
    *,
    sm_scale: Optional[float] = None,
    return_artifacts: bool = False,
    preprocess_cache: Optional[PreprocessCache] = None,
) -> torch.Tensor | tuple[torch.Tensor, FakeQuantArtifacts]:
    """Fake-quant attention with FP8/MXFP8 Q/K/V (and optional P requant).

    ``q, k, v``: ``(B, S, H, D)``, ``D in {64, 128}``, bf16/fp16/fp32 on the GPU.
    Returns ``(B, S, H, D)`` in the input dtype (plus artifacts if requested).
    """
    if cfg is None:
        cfg = QuantConfig()
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(
            f"q/k/v shapes must match; got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}"
        )
    if q.ndim != 4:
        raise ValueError(f"q/k/v must be 4-D (B,S,H,D); got {q.shape}")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q/k/v must live on CUDA")
    out_dtype = q.dtype
    if out_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported dtype {out_dtype}")
    sdpa_dtype = torch.float16 if out_dtype == torch.float16 else torch.bfloat16
    b, s, h, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if cfg.blasst_lambda is not None and not cfg.p_requant:
        raise ValueError("BLASST skip/fill requires cfg.p_requant=True")

    if preprocess_cache is not None:
        pc = preprocess_cache
        if (
            pc.smoothing != cfg.smoothing
            or pc.q_kmeans_k != cfg.q_kmeans_k
            or pc.q_smooth_block_size != cfg.q_smooth_block_size
            or pc.v_smooth_mode != cfg.v_smooth_mode
            or pc.v_smooth_block_size != cfg.v_smooth_block_size
            or pc.v_kmeans_k != cfg.v_kmeans_k
        ):
            raise ValueError("preprocess_cache does not match cfg's smoothing/kmeans/v_smooth settings")
        prep = _prep_from_cache(pc)
    else:
        prep = _lazy_preprocess(q, k, v, cfg)

    if cfg.p_requant:
        o = _p_requant_hip(prep, cfg, sm_scale, out_dtype)
    else:
        o = _sdpa_hip(prep, cfg, sm_scale, out_dtype, sdpa_dtype)

    if return_artifacts:
        km = prep.q_km_result if prep.q_km_result is not None else _kmeans_result(q.contiguous(), prep.q_km)
        art = FakeQuantArtifacts(qm=prep.qm, kmeans=km, q_eff_dtype=sdpa_dtype, p_requant=cfg.p_requant,
                                 qk_hadamard=cfg.qk_hadamard)
        return o, art
    return o


def reference_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    sm_scale: Optional[float] = None,
) -> torch.Tensor:
    """Unquantised reference attention (fp32 softmax, contiguous operands)."""
    if q.ndim != 4:
        raise ValueError(f"q/k/v must be (B,S,H,D); got {q.shape}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    perm = (0, 2, 1, 3)
    o = _attention_fp32(q.permute(*perm), k.permute(*perm), v.permute(*perm), sm_scale)
    return o.to(q.dtype).permute(*perm).contiguous()


__all__ = ["FakeQuantArtifacts", "fake_quant_attention", "reference_attention", "PreprocessCache",
           "prepare_for_attention"]
