"""CPU restatement of ``fake_quant_attention`` end to end (test infrastructure only).

Follows ``attention.py`` of the reference:

* ``preprocess``           -- ``attention.py:166-239`` (Q k-means, K smoothing,
                              Q group mean, V k-means + K co-permute, V smoothing);
* ``quant_qk_deq``         -- ``attention.py:89-121, 531-535`` (optional Hadamard
                              on the quantiser inputs, quant, dequant to bf16);
* ``p_requant_path``       -- ``attention.py:505-639`` (V kind marshalling,
                              rowmax estimate, P mode, kernel call);
* ``sdpa_path``            -- ``attention.py:247-321``;
* ``fake_quant_attention`` -- ``attention.py:706-806`` (guards, inverse Q gather);
* ``prepare_qkv``          -- the legacy pipeline ``pipeline.py:42-110`` (Q k-means,
                              smoothing with the qm.K_s correction, Hadamard on the
                              smoothed tensors, then quantisation).

``cfg`` is any object with the ``QuantConfig`` fields.  All tensors are CPU.

Pinned by ``tests/test_oracle_pipeline.py``: Q k-means reorder + inverse gather
is a bitwise row permutation when per-row MX scales make quantisation
order-independent; V k-means with the K co-permutation only reorders the key
sum under a fixed row max; the SDPA path equals torch SDPA on the dequantised
tensors.  The functions it composes are pinned in their own modules.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import attention as oattn
from . import hadamard as ohad
from . import kmeans as okm
from . import preprocess as opre
from . import quant as oq


def preprocess(q, k, v, cfg):
    q_work, k_work, v_work = q.contiguous(), k.contiguous(), v.contiguous()
    q_km = None
    if cfg.q_kmeans_k is not None:
        q_km = okm.kmeans_reorder_tokens(q_work, n_clusters=cfg.q_kmeans_k,
                                         max_iters=cfg.q_kmeans_iters, seed=cfg.q_kmeans_seed)
        q_work = q_km["tensor_reordered"]
    qm = None
    if cfg.smoothing == "off":
        pass
    elif cfg.smoothing == "k_only":
        k_work, _ = opre.smooth_k(k_work)
    elif cfg.smoothing == "full":
        k_work, _ = opre.smooth_k(k_work)
        q_work, qm = opre.group_mean_q(q_work, block_q=cfg.q_smooth_block_size)
    else:
        raise ValueError(f"unsupported smoothing: {cfg.smoothing!r}")
    v_km = None
    if cfg.v_kmeans_k is not None:
        v_km = okm.kmeans_reorder_tokens(v_work, n_clusters=cfg.v_kmeans_k,
                                         max_iters=cfg.v_kmeans_iters, seed=cfg.v_kmeans_seed)
        v_work = v_km["tensor_reordered"]
        k_work = okm.apply_kv_permutation(k_work, v_km["order"])
    v_alpha = None
    if cfg.v_smooth_mode == "per_block":
        v_work, v_alpha = opre.smooth_v_per_block(v_work, block_s=cfg.v_smooth_block_size)
    elif cfg.v_smooth_mode != "off":
        raise ValueError(f"unsupported v_smooth_mode: {cfg.v_smooth_mode!r}")
    return q_work, k_work, v_work, qm, v_alpha, q_km, v_km


def quant_qk(t, cfg):
    if cfg.qk_quant == "fp8_block":
        c, s = oq.fp8_block_quant(t, cfg.fp8_block_size)
        return c, s, ("fp8_block", cfg.fp8_block_size)
    if cfg.qk_quant == "mxfp8":
        c, s = oq.mxfp8_qk_quant(t, cfg.mxfp8_block_size)
        return c, s, ("mxfp8", cfg.mxfp8_block_size)
    raise ValueError(f"unsupported qk_quant: {cfg.qk_quant!r}")


def dequant_qk(c, s, meta, dtype):
    if meta[0] == "fp8_block":
        return oq.fp8_block_dequant(c, s, meta[1], dtype=dtype)
    return oq.mxfp8_qk_dequant(c, s, meta[1], dtype=dtype)


def quant_v(t, cfg):
    if cfg.v_quant == "fp8_channel":
        c, s = oq.fp8_per_channel_quant(t)
        return c, s, ("fp8_channel", 0)
    if cfg.v_quant == "fp8_block":
        c, s = oq.fp8_block_quant(t, cfg.v_fp8_block_size)
        return c, s, ("fp8_block", cfg.v_fp8_block_size)
    if cfg.v_quant == "mxfp8":
        c, s = oq.mxfp8_v_quant(t, cfg.v_mxfp8_block_size)
        return c, s, ("mxfp8", cfg.v_mxfp8_block_size)
    raise ValueError(f"unsupported v_quant: {cfg.v_quant!r}")


def dequant_v(c, s, meta, dtype):
    if meta[0] == "fp8_channel":
        return oq.fp8_per_channel_dequant(c, s, dtype=dtype)
    if meta[0] == "fp8_block":
        return oq.fp8_block_dequant(c, s, meta[1], dtype=dtype)
    return oq.mxfp8_v_dequant(c, s, meta[1], dtype=dtype)


def qk_quant_inputs(q_work, k_work, cfg):
    if not cfg.qk_hadamard:
        return q_work, k_work
    return ohad.apply_qk_hadamard(q_work, k_work, random_sign=cfg.qk_hadamard_random_sign,
                                  seed=cfg.qk_hadamard_seed)


def p_requant_path(q_work, k_work, v_work, qm, v_alpha, cfg, sm_scale, out_dtype, rows=None,
                   return_blasst_stats=False, qk_dequant_dtype=torch.bfloat16, scores_log2=None,
                   return_debug=False, force_codes=None, rowmax_log2=None, rowmax_init=None):
    """``qk_dequant_dtype=torch.bfloat16`` is the reference (attention.py:534-535);
    ``torch.float32`` keeps the dequantised Q/K exact and is used only to measure
    how sensitive the reference output is to that rounding.  ``scores_log2``,
    ``return_debug`` and ``force_codes`` are passed to ``attention.attention``
    (rows in the reordered order of the work tensors); ``rowmax_log2``
    (B,H,G), when given, replaces the qm_k row-max estimate (log2 units, one
    value per Q group) -- used with ``scores_log2`` to replay the reference
    algorithm on another implementation's scores and estimate.  ``rowmax_init``
    (B,H,S), natural-log units, rows in the work order: the reference kernel's
    rowmax_init_bhs (attention_triton.py:127-130), passed to the attention."""
    b, s, h, d = q_work.shape
    qi, ki = qk_quant_inputs(q_work, k_work, cfg)
    qc, qs, qmeta = quant_qk(qi, cfg)
    kc, ks, kmeta = quant_qk(ki, cfg)
    q_deq = dequant_qk(qc, qs, qmeta, qk_dequant_dtype)
    k_deq = dequant_qk(kc, ks, kmeta, qk_dequant_dtype)
    vc, vs, vmeta = quant_v(v_work, cfg)
    v_block_scale, v_block_size = None, 0
    if vmeta[0] == "fp8_channel":
        v_bf = oq.decode(vc).to(torch.bfloat16)
        v_scale = vs.float()
    elif vmeta[0] == "fp8_block":
        v_bf = oq.decode(vc).to(torch.bfloat16)
        v_scale = torch.ones(b, h, d)
        v_block_scale, v_block_size = vs.float(), vmeta[1]
    else:
        v_bf = dequant_v(vc, vs, vmeta, torch.bfloat16)
        v_scale = torch.ones(b, h, d)
    perm = (0, 2, 1, 3)
    k_smooth = qm_arg = None
    if qm is not None:
        k_smooth = k_work.to(torch.bfloat16).permute(*perm).contiguous()
        qm_arg = qm.float()
    rowmax_est = None
    if cfg.rowmax_mode == "qm_k":
        if qm is None:
            raise ValueError("rowmax_mode='qm_k' requires smoothing='full' so qm exists")
        if rowmax_log2 is None:
            rowmax_est = oattn.estimate_rowmax_qm_k(qm, k_work, block_q=cfg.q_smooth_block_size,
                                                    sm_scale=sm_scale)
        else:
            rowmax_est = (rowmax_log2.float() / torch.tensor(oattn.LOG2E, dtype=torch.float32)).repeat_interleave(
                cfg.q_smooth_block_size, dim=2).contiguous()
    elif cfg.rowmax_mode != "online":
        raise ValueError(f"unsupported rowmax_mode: {cfg.rowmax_mode!r}")
    p_mode = cfg.p_quant
    if p_mode == "auto":
        p_mode = "mx" if vmeta[0] == "mxfp8" else "elementwise"
    res = oattn.attention(
        q_deq.permute(*perm).contiguous(), k_deq.permute(*perm).contiguous(),
        v_bf.permute(*perm).contiguous(), v_scale,
        sm_scale=sm_scale, p_max_offset=int(cfg.p_max_offset),
        block_m=cfg.p_requant_block_m, block_n=cfg.p_requant_block_n,
        v_alpha=v_alpha, v_smooth_block=cfg.v_smooth_block_size if v_alpha is not None else 0,
        k_smooth=k_smooth, qm=qm_arg, q_smooth_block=cfg.q_smooth_block_size if qm is not None else 0,
        v_block_scale=v_block_scale, v_block_size=v_block_size, p_quant_mode=p_mode,
        rowmax_est=rowmax_est, blasst_lambda=cfg.blasst_lambda, blasst_fill_mode=cfg.blasst_fill,
        blasst_fill_alpha=cfg.blasst_fill_alpha, blasst_uta_bins=cfg.blasst_uta_bins,
        return_blasst_stats=return_blasst_stats, rows=rows, return_debug=return_debug,
        scores_log2=scores_log2, force_codes=force_codes, rowmax_init=rowmax_init)
    res = list(res) if isinstance(res, tuple) else [res]
    res[0] = res[0].permute(*perm).contiguous().to(out_dtype)
    return res[0] if len(res) == 1 else tuple(res)


def sdpa_path(q_work, k_work, v_work, qm, v_alpha, cfg, sm_scale, sdpa_dtype):
    b, s, h, d = q_work.shape
    qi, ki = qk_quant_inputs(q_work, k_work, cfg)
    qc, qs, qmeta = quant_qk(qi, cfg)
    kc, ks, kmeta = quant_qk(ki, cfg)
    vc, vs, vmeta = quant_v(v_work, cfg)
    q_deq = dequant_qk(qc, qs, qmeta, sdpa_dtype)
    k_deq = dequant_qk(kc, ks, kmeta, sdpa_dtype)
    v_deq = dequant_v(vc, vs, vmeta, sdpa_dtype)
    if v_alpha is not None:
        v_deq = v_deq + v_alpha.repeat_interleave(cfg.v_smooth_block_size, dim=1).to(sdpa_dtype)
    perm = (0, 2, 1, 3)
    if qm is None:
        o = F.scaled_dot_product_attention(q_deq.permute(*perm).float(), k_deq.permute(*perm).float(),
                                           v_deq.permute(*perm).float(), scale=sm_scale)
        return o.to(sdpa_dtype).permute(*perm).contiguous()
    block_q = cfg.q_smooth_block_size
    qb = q_deq.permute(*perm).float()
    qmb = qm.permute(*perm).float()
    kb = k_deq.permute(*perm).float()
    ksb = k_work.permute(*perm).float()
    vb = v_deq.permute(*perm).float()
    grp = torch.arange(s) // block_q
    # attention.py:314: a matmul of the sdpa-dtype operands, its output rounded
    # to that dtype, then scaled in fp32
    s_main = torch.matmul(q_deq.permute(*perm).contiguous(),
                          k_deq.permute(*perm).transpose(-2, -1).contiguous()).float() * sm_scale
    s_corr = torch.matmul(qmb[:, :, grp], ksb.transpose(-2, -1)) * sm_scale
    p = torch.softmax(s_main + s_corr, dim=-1).to(sdpa_dtype).float()
    return torch.matmul(p, vb).to(sdpa_dtype).permute(*perm).contiguous()


def fake_quant_attention(q, k, v, cfg, *, sm_scale=None, return_blasst_stats=False,
                         qk_dequant_dtype=torch.bfloat16, scores_log2=None, return_debug=False,
                         force_codes=None, rowmax_log2=None, rowmax_init=None):
    """Output in the caller's row order.  With ``return_debug`` the debug dict of
    ``attention.attention`` (reordered row order) follows, plus ``"order"``
    (the Q k-means order, or None)."""
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q/k/v shapes must match")
    out_dtype = q.dtype
    sdpa_dtype = torch.float16 if out_dtype == torch.float16 else torch.bfloat16
    b, s, h, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if cfg.blasst_lambda is not None and not cfg.p_requant:
        raise ValueError("BLASST skip/fill requires cfg.p_requant=True")
    q_work, k_work, v_work, qm, v_alpha, q_km, _ = preprocess(q, k, v, cfg)
    stats = dbg = None
    if cfg.p_requant:
        r = p_requant_path(q_work, k_work, v_work, qm, v_alpha, cfg, sm_scale, out_dtype,
                           return_blasst_stats=return_blasst_stats, qk_dequant_dtype=qk_dequant_dtype,
                           scores_log2=scores_log2, return_debug=return_debug, force_codes=force_codes,
                           rowmax_log2=rowmax_log2, rowmax_init=rowmax_init)
        r = list(r) if isinstance(r, tuple) else [r]
        o = r.pop(0)
        stats = r.pop(0) if return_blasst_stats else None
        dbg = r.pop(0) if return_debug else None
        if dbg is not None:
            dbg["order"] = q_km["order"] if q_km is not None else None
    else:
        o = sdpa_path(q_work, k_work, v_work, qm, v_alpha, cfg, sm_scale, sdpa_dtype).to(out_dtype)
    if dbg is not None:
        dbg["flip_allowance_nhd"] = dbg["flip_allowance"].permute(0, 2, 1, 3).contiguous()
    if q_km is not None:
        inv = q_km["inverse_order"]

        def unreorder(t):
            tb = t.permute(0, 2, 1, 3).reshape(b * h, s, d)
            return torch.gather(tb, 1, inv.unsqueeze(-1).expand(-1, -1, d)).reshape(b, h, s, d).permute(
                0, 2, 1, 3).contiguous()

        o = unreorder(o)
        if dbg is not None:
            dbg["flip_allowance_nhd"] = unreorder(dbg["flip_allowance_nhd"])
    out = [o] + ([stats] if return_blasst_stats else []) + ([dbg] if return_debug else [])
    return out[0] if len(out) == 1 else tuple(out)


def prepare_qkv(q, k, v, cfg):
    """``pipeline.py:42-110``: returns a dict with the fields of PreparedQKV
    (codes as uint8, scales, qm, k_mean, correction (B, G, H, S) fp32 before
    the cast to ``cfg.correction_dtype``, the k-means result)."""
    q_work, k_work, v_work = q.contiguous(), k.contiguous(), v.contiguous()
    km = None
    if cfg.q_kmeans_k is not None:
        km = okm.kmeans_reorder_tokens(q_work, n_clusters=cfg.q_kmeans_k, max_iters=cfg.q_kmeans_iters,
                                       seed=cfg.q_kmeans_seed)
        q_work = km["tensor_reordered"]
    qm = k_mean = corr = None
    if cfg.smoothing == "k_only":
        k_work, k_mean = opre.smooth_k(k_work)
    elif cfg.smoothing == "full":
        k_work, k_mean = opre.smooth_k(k_work)
        q_work, qm = opre.group_mean_q(q_work, block_q=cfg.q_smooth_block_size)
        corr = torch.einsum("bqhd,bshd->bqhs", qm.double(), k_work.double())   # exact-ish; fp32 in the reference
    elif cfg.smoothing != "off":
        raise ValueError(f"unsupported smoothing mode: {cfg.smoothing!r}")
    if cfg.qk_hadamard:
        q_work, k_work = ohad.apply_qk_hadamard(q_work, k_work, random_sign=cfg.qk_hadamard_random_sign,
                                                seed=cfg.qk_hadamard_seed)
    qc, qs, _ = quant_qk(q_work, cfg)
    kc, ks, _ = quant_qk(k_work, cfg)
    vc, vs, _ = quant_v(v_work, cfg)
    return {"q": qc, "k": kc, "v": vc, "q_scale": qs, "k_scale": ks, "v_scale": vs, "qm": qm, "k_mean": k_mean,
            "correction": corr, "kmeans": km}
