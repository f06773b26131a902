"""Wan2.1 attention hook: self-attention through ``fake_quant_attention``.

Replaces ``wan.modules.attention.attention`` / ``flash_attention`` (and the
name ``wan.modules.model`` imported) with :func:`fake_or_sdpa_attention`,
the call boundary of the reference hook (``bench/wan_attention_hook.py:
203-327``):

* self-attention -- ``Lq == Lk`` and ``Lq > 1024`` (video tokens; Wan's text
  context is 512) -- runs ``fake_quant_attention`` under the active
  ``QuantConfig``, after padding the sequence to the LCM of the block sizes
  (Q zero rows, K/V repeating their last row; ``wan.pad_qkv``), and slices
  the output back to ``Lq``;
* cross-attention, and self-attention while the active config is ``None``
  (``NO_QUANT``), run plain scaled-dot-product attention.

Optional diagnostics, switched by the same environment variables as the
reference hook (``:60-186``):

* ``WAN_ATTENTION_DUMP_DIR`` (+ ``WAN_ATTENTION_DUMP_CALLS`` = comma list of
  call indices, or ``WAN_ATTENTION_DUMP_LIMIT``, default 1): save the
  self-attention inputs as ``call_NNN.pt`` holding CPU tensors
  ``{"query", "key", "value"}`` and the call record;
* ``WAN_ATTENTION_COMPARE_SDPA=1``: record mse / cosine / max-abs of the
  output against exact attention;
* ``WAN_ATTENTION_COMPARE_ONLINE_ROWMAX=1`` (``rowmax_mode="qm_k"`` only):
  record the same against ``rowmax_mode="online"`` on a shared preprocess.

The exact attention of the SDPA fallback and of the comparison is computed
in float32 (contiguous operands) and rounded to the input dtype.
"""

from __future__ import annotations

import math
import os
import threading
from dataclasses import replace
from pathlib import Path
from typing import Optional

import torch
import torch.nn.functional as F

from .attention import PreprocessCache, fake_quant_attention, prepare_for_attention
from .config import QuantConfig
from .wan import pad_length, pad_qkv

# Sentinel for "no fake quant, exact attention everywhere".
NO_QUANT: Optional[QuantConfig] = None

SELF_ATTENTION_MIN_LEN = 1024

_state_lock = threading.Lock()
_current_cfg: Optional[QuantConfig] = None
_call_log: list = []
_installed: dict = {}


def set_quant_cfg(cfg: Optional[QuantConfig]) -> None:
    """Set the active config (``None`` = exact attention) and clear the call log."""
    global _current_cfg
    with _state_lock:
        _current_cfg = cfg
        _call_log.clear()


def get_quant_cfg() -> Optional[QuantConfig]:
    with _state_lock:
        return _current_cfg


def get_call_log() -> list:
    """A copy of the per-call records since the last ``set_quant_cfg``."""
    with _state_lock:
        return list(_call_log)


def _log_call(record: dict) -> None:
    with _state_lock:
        _call_log.append(record)


def is_self_attention(lq: int, lk: int) -> bool:
    return lq == lk and lq > SELF_ATTENTION_MIN_LEN


def exact_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, softmax_scale: float,
                    dropout_p: float = 0.0, causal: bool = False) -> torch.Tensor:
    """Scaled-dot-product attention of NHD tensors, float32 inside, NHD out (float32)."""
    qb = q.transpose(1, 2).float().contiguous()
    kb = k.transpose(1, 2).float().contiguous()
    vb = v.transpose(1, 2).float().contiguous()
    out = F.scaled_dot_product_attention(qb, kb, vb, dropout_p=dropout_p, is_causal=causal, scale=softmax_scale)
    return out.transpose(1, 2).contiguous()


def _agreement(out: torch.Tensor, ref: torch.Tensor) -> dict:
    a = out.float().flatten()
    b = ref.float().flatten()
    diff = a - b
    an = torch.linalg.vector_norm(a)
    bn = torch.linalg.vector_norm(b)
    return {
        "mse": float(diff.pow(2).mean().item()),
        "cosine": float((torch.dot(a, b) / torch.clamp(an * bn, min=1e-12)).item()),
        "max_abs": float(diff.abs().max().item()),
        "out_norm": float(an.item()),
        "ref_norm": float(bn.item()),
        "out_has_nan": bool(torch.isnan(out).any().item()),
        "out_has_inf": bool(torch.isinf(out).any().item()),
    }


def _maybe_dump_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, record: dict) -> None:
    dump_dir = os.environ.get("WAN_ATTENTION_DUMP_DIR")
    if not dump_dir:
        return
    with _state_lock:
        call_idx = len(_call_log)
        dumped = sum(1 for r in _call_log if r.get("dumped_qkv"))
    wanted = os.environ.get("WAN_ATTENTION_DUMP_CALLS")
    if wanted:
        if call_idx not in {int(x) for x in wanted.split(",") if x.strip()}:
            return
    elif dumped >= int(os.environ.get("WAN_ATTENTION_DUMP_LIMIT", "1")):
        return
    if dumped >= int(os.environ.get("WAN_ATTENTION_DUMP_LIMIT", "1000000")):
        return
    out_dir = Path(dump_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    path = out_dir / f"call_{call_idx:03d}.pt"
    torch.save({"query": q.detach().cpu(), "key": k.detach().cpu(), "value": v.detach().cpu(),
                "record": dict(record)}, path)
    record["dumped_qkv"] = str(path)


def load_qkv_dump(path, device=None, dtype=torch.bfloat16):
    """(q, k, v) of a dump written by this hook or the reference hook.

    Only tensors and plain containers are accepted (``weights_only=True``).
    """
    obj = torch.load(path, map_location="cpu", weights_only=True)
    return tuple(obj[n].to(device=device, dtype=dtype) for n in ("query", "key", "value"))


def fake_or_sdpa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_lens: Optional[torch.Tensor] = None,
    k_lens: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    softmax_scale: Optional[float] = None,
    q_scale: Optional[float] = None,
    causal: bool = False,
    window_size: tuple = (-1, -1),
    deterministic: bool = False,
    dtype: torch.dtype = torch.bfloat16,
    fa_version=None,
    version=None,
) -> torch.Tensor:
    """Drop-in for Wan's ``attention`` / ``flash_attention`` (NHD ``(B, L, N, C)``).

    Same arguments as the function it replaces; ``q_lens``/``k_lens``,
    ``window_size``, ``deterministic`` and the version selectors are accepted
    and ignored, as in the reference hook (batch-1 evaluation).
    """
    b, lq, nh, c = q.shape
    lk = k.shape[1]
    cfg = get_quant_cfg()
    self_attn = is_self_attention(lq, lk)

    half = (torch.float16, torch.bfloat16)
    if q.dtype not in half:
        q = q.to(dtype)
    if k.dtype not in half:
        k = k.to(dtype)
    if v.dtype not in half:
        v = v.to(dtype)
    if q_scale is not None:
        q = q * q_scale
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(c)

    if self_attn and cfg is not None:
        pad = pad_length(lq, cfg) - lq
        record = {"kind": "self-fq", "Lq": lq, "Lk": lk, "D": c, "H": nh, "pad": pad}
        _maybe_dump_qkv(q, k, v, record)
        compare_online = (os.environ.get("WAN_ATTENTION_COMPARE_ONLINE_ROWMAX") == "1"
                          and cfg.rowmax_mode == "qm_k")
        qp, kp, vp, _ = pad_qkv(q, k, v, cfg)
        cache: Optional[PreprocessCache] = prepare_for_attention(qp, kp, vp, cfg) if compare_online else None
        out = fake_quant_attention(qp, kp, vp, cfg, sm_scale=softmax_scale, preprocess_cache=cache)[:, :lq]
        if os.environ.get("WAN_ATTENTION_COMPARE_SDPA") == "1":
            ref = exact_attention(q, k, v, softmax_scale=softmax_scale, dropout_p=dropout_p, causal=causal)
            record["compare_sdpa"] = _agreement(out, ref)
        if compare_online:
            ref = fake_quant_attention(qp, kp, vp, replace(cfg, rowmax_mode="online"), sm_scale=softmax_scale,
                                       preprocess_cache=cache)[:, :lq]
            rec = _agreement(out, ref)
            rec["ref_has_nan"] = bool(torch.isnan(ref).any().item())
            rec["ref_has_inf"] = bool(torch.isinf(ref).any().item())
            record["compare_online_rowmax"] = rec
        _log_call(record)
        return out.to(q.dtype)

    out = exact_attention(q, k, v, softmax_scale=softmax_scale, dropout_p=dropout_p, causal=causal)
    _log_call({"kind": "self-sdpa" if self_attn else "cross-sdpa", "Lq": lq, "Lk": lk, "D": c, "H": nh})
    return out.to(q.dtype)


def install_hook(attention_module=None, model_module=None) -> None:
    """Patch Wan's attention entry points (idempotent).

    By default imports ``wan.modules.attention`` and ``wan.modules.model``
    (``ImportError`` when Wan is not installed); modules can also be passed
    in directly.  Patches ``attention`` and ``flash_attention`` of the first
    and ``flash_attention`` of the second, which imports it by name.
    """
    if attention_module is None:
        import wan.modules.attention as attention_module  # noqa: F811
    if model_module is None:
        import wan.modules.model as model_module  # noqa: F811
    key = (id(attention_module), id(model_module))
    if _installed.get(key):
        return
    attention_module.attention = fake_or_sdpa_attention
    attention_module.flash_attention = fake_or_sdpa_attention
    model_module.flash_attention = fake_or_sdpa_attention
    _installed[key] = True


__all__ = ["install_hook", "set_quant_cfg", "get_call_log", "NO_QUANT", "fake_or_sdpa_attention",
           "load_qkv_dump"]
