"""``QuantConfig``: the knob surface of the fake-quant attention path.

Field names, types, defaults and meanings are those of the reference
(``src/low_bit_fake_quant/config.py:35-122``) so existing callers construct the
same object and get the same semantics.  Only the execution backend differs:
every field is consumed by hand-written gfx950 kernels instead of Triton.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch

QKQuant = Literal["fp8_block", "mxfp8"]
# V quantization scheme:
#   fp8_channel: one FP32 scale per (B, H, D), shared across S.
#   fp8_block:   one FP32 scale per (B, S/v_fp8_block_size, H).
#   mxfp8:       one power-of-two scale per (B, S/v_mxfp8_block_size, H, D).
VQuant = Literal["fp8_channel", "fp8_block", "mxfp8"]
Smoothing = Literal["off", "k_only", "full"]
VSmoothMode = Literal["off", "per_block"]
# P quantization: auto -> mx when v_quant == "mxfp8", else elementwise.
PQuant = Literal["auto", "elementwise", "mx", "dynamic"]
RowmaxMode = Literal["online", "qm_k"]
# BLASST fill for skipped row/K-blocks.  Probe spellings such as
# "mean_a1.5" or "uta16_a1.5" are accepted, so this stays a plain string.
BlasstFill = str


@dataclass(frozen=True)
class QuantConfig:
    """Configuration for Q/K/V fake-quant preprocessing and attention.

    Defaults: Q/K FP32-scale block FP8 (block 128), V per-channel FP8, full
    smoothing, Q k-means with 32 clusters, P requantised to FP8 with
    ``p_max_offset=8``.
    """

    qk_quant: QKQuant = "fp8_block"
    v_quant: VQuant = "fp8_channel"
    smoothing: Smoothing = "full"
    q_smooth_block_size: int = 256
    q_kmeans_k: int | None = 32
    q_kmeans_iters: int = 10
    q_kmeans_seed: int = 0
    # Orthonormal (optionally random-sign) Hadamard rotation of Q/K along D,
    # applied to the quantiser inputs only.
    qk_hadamard: bool = False
    qk_hadamard_random_sign: bool = True
    qk_hadamard_seed: int = 0
    fp8_block_size: int = 128         # Q/K fp8_block: one scale per (B, S/blk, H)
    mxfp8_block_size: int = 32        # Q/K mxfp8: one scale per (B, S, H, D/blk)
    v_fp8_block_size: int = 64        # V fp8_block: one scale per (B, S/blk, H)
    v_mxfp8_block_size: int = 64      # V mxfp8: one scale per (B, S/blk, H, D)
    p_quant: PQuant = "auto"
    # "online": exact running row max.  "qm_k": per-row estimate
    # max_n(qm[group] . K_smooth[n]) (requires smoothing="full").
    rowmax_mode: RowmaxMode = "online"
    # P MX block along N; 0 means "use v_mxfp8_block_size".
    p_mx_block_n: int = 0
    p_max_offset: int = 8
    correction_dtype: torch.dtype = torch.float16
    # Cast P to FP8 e4m3fn before PV.  False: dequantised Q/K/V through SDPA.
    p_requant: bool = True
    # Kept for API compatibility (the reference's legacy torch path chunk).
    p_requant_q_chunk: int = 512
    # Row / key block sizes of the P-requant attention.  block_n fixes the
    # granularity of the mx/dynamic P scales and of the BLASST predicate.
    p_requant_block_m: int = 64
    p_requant_block_n: int = 64
    # BLASST skip/fill.  None disables it; otherwise lambda in (0, 1).
    blasst_lambda: float | None = None
    blasst_fill: BlasstFill = "zero"
    blasst_fill_alpha: float = 1.0
    blasst_uta_bins: int = 16
    # V per-block mean smoothing (mean folded back through a C accumulator).
    v_smooth_mode: VSmoothMode = "off"
    v_smooth_block_size: int = 64
    # V k-means token reorder (K co-permuted with the same order).
    v_kmeans_k: int | None = None
    v_kmeans_iters: int = 10
    v_kmeans_seed: int = 0
