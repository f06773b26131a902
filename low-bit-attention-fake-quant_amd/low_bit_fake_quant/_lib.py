"""ctypes binding of ``liblbfq_hip.so`` (declarations: ``include/lbfq.h``).

The shared library is the only compute backend of this package: there is no
CPU or Triton fallback.  If it is missing, or no ROCm GPU is visible, every
entry point raises.  ``torch`` is imported first so the library resolves to
the HIP runtime torch already loaded (one runtime per process).
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblbfq_hip.so")

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

SUB_NONE, SUB_COLVEC, SUB_BLOCKVEC = 0, 1, 2
Q_NONE, Q_FP8_BLOCK, Q_CHANNEL, Q_MX_QK, Q_MX_V, Q_CHANNEL_AMAX = range(6)
LAYOUT_NHD, LAYOUT_BHSD, LAYOUT_BHDS = 0, 1, 2
DQ_BLOCK, DQ_CHANNEL, DQ_MX_QK, DQ_MX_V = range(4)

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_vp = ctypes.c_void_p


class RowTileParams(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_dtype", _i32),
        ("B", _i64), ("S", _i64), ("H", _i64), ("D", _i64),
        ("R", _i32),
        ("gather", _vp),
        ("sub_mode", _i32), ("sub", _vp),
        ("sub_block", _i32),
        ("smoothed", _vp),
        ("hadamard", _i32), ("signs", _vp),
        ("had_scale", _f32),
        ("quant_mode", _i32),
        ("codes", _vp), ("codes_layout", _i32),
        ("codes_spitch", _i64),
        ("scale", _vp),
        ("sc_b", _i64), ("sc_s", _i64), ("sc_h", _i64), ("sc_d", _i64),
        ("amax_table", _vp),
        ("mx_block", _i32),
        ("smoothed_stage", _i32),
        ("scale_e8m0", _i32),
    ]


class AttnParams(ctypes.Structure):
    _fields_ = [
        ("B", _i64), ("H", _i64), ("S", _i64), ("D", _i64),
        ("s_pitch", _i64),
        ("q_codes", _vp), ("k_codes", _vp), ("v_codes_t", _vp),
        ("qk_mx", _i32),
        ("q_scale", _vp),
        ("k_scale", _vp),
        ("qk_block", _i32),
        ("v_kind", _i32), ("v_scale", _vp),
        ("v_block", _i32),
        ("p_mode", _i32),
        ("sm_scale", _f32),
        ("p_max_offset", _i32),
        ("block_m", _i32),
        ("qk_bias", _vp),
        ("q_group", _i32),
        ("rowmax_est", _vp),
        ("rowmax_dynamic", _i32),
        ("v_alpha", _vp),
        ("v_smooth_block", _i32),
        ("blasst_lambda", _f32),
        ("blasst_fill", _i32),
        ("blasst_fill_alpha", _f32),
        ("blasst_uta_bins", _i32),
        ("blasst_stats", _vp),
        ("out", _vp), ("out_dtype", _i32),
        ("out_row_map", _vp),
        ("blasst_row_skips", _vp),
        ("blasst_wave_tiles", _vp),
        ("v_tile_colsum", _vp),
        ("block_n", _i32),
        ("rowmax_init", _vp),
    ]


class RowmaxCountParams(ctypes.Structure):
    _fields_ = [
        ("B", _i64), ("H", _i64), ("S", _i64), ("D", _i64), ("s_pitch", _i64),
        ("q_codes", _vp), ("k_codes", _vp),
        ("q_scale", _vp), ("k_scale", _vp),
        ("qk_block", _i32),
        ("bias", _vp),
        ("rowmax_est", _vp),
        ("q_group", _i32),
        ("sm_scale", _f32),
        ("up_threshold_log2", _f32), ("down_threshold_log2", _f32), ("mass_floor", _f32),
        ("down_always", _i32), ("use_estimate", _i32),
        ("counters", _vp),
    ]


class BlasstAttendParams(ctypes.Structure):
    _fields_ = [
        ("S", _i64), ("H", _i64), ("D", _i64),
        ("q", _vp), ("k", _vp), ("v", _vp),
        ("sm_scale", _f32),
        ("mode", _i32),
        ("round_p_bf16", _i32),
        ("final_max", _vp),
        ("keep", _vp),
        ("out", _vp),
        ("dropped", _vp),
        ("p_counts", _vp),
        ("p_sqerr", _vp),
    ]


class SdpaDequantParams(ctypes.Structure):
    _fields_ = [
        ("B", _i64), ("H", _i64), ("S", _i64), ("D", _i64), ("s_pitch", _i64),
        ("q_codes", _vp), ("k_codes", _vp), ("v_codes_t", _vp),
        ("qk_mx", _i32), ("q_scale", _vp), ("k_scale", _vp), ("qk_block", _i32),
        ("v_kind", _i32), ("v_scale", _vp), ("v_block", _i32),
        ("v_alpha", _vp), ("v_smooth_block", _i32),
        ("sdpa_dtype", _i32),
        ("q_out", _vp), ("k_out", _vp), ("v_t_out", _vp),
    ]


class SdpaParams(ctypes.Structure):
    _fields_ = [
        ("B", _i64), ("H", _i64), ("S", _i64), ("D", _i64), ("s_pitch", _i64),
        ("q", _vp), ("k", _vp), ("v_t", _vp),
        ("sdpa_dtype", _i32),
        ("sm_scale", _f32),
        ("qk_bias", _vp),
        ("groups", _i64),
        ("q_group", _i32),
        ("out", _vp), ("out_dtype", _i32),
        ("out_row_map", _vp),
    ]


# name -> (restype, argtypes)
_SIGS = {
    "lbfq_last_error": (ctypes.c_char_p, []),
    "lbfq_rowtile": (_i32, [ctypes.POINTER(RowTileParams), _vp]),
    "lbfq_colsum": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i32, _vp, _i32, _vp, _vp, _vp]),
    "lbfq_colsum_finalize": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "lbfq_fill_u32": (_i32, [_vp, _i64, ctypes.c_uint32, _vp]),
    "lbfq_dequant": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _vp, _i32, _vp]),
    "lbfq_kmeans_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "lbfq_kmeans": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i32, _i32, ctypes.c_uint64, _vp, _vp, _vp, _vp,
                           _vp]),
    "lbfq_kmeans_noalloc_max_workspace_bytes": (_i64, []),
    "lbfq_kmeans_noalloc": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i32, _i32, ctypes.c_uint64, _vp, _vp, _vp,
                                   _vp]),
    "lbfq_qmk": (_i32, [_vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp, _i64, _vp, _vp, _vp]),
    "lbfq_qmk_kquant": (_i32, [_vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp, _i64, _vp, _vp,
                               _vp, _i64, _vp, _i64, _vp]),
    "lbfq_attention_fwd": (_i32, [ctypes.POINTER(AttnParams), _vp]),
    "lbfq_attention_scores": (_i32, [ctypes.POINTER(AttnParams), _vp, _i64, _vp, _vp]),
    "lbfq_v_tile_colsum": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _i32, _vp, _vp]),
    "lbfq_p_requant_rows": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp,
                                   ctypes.c_double, _i32, _vp]),
    "lbfq_rowmax_count": (_i32, [ctypes.POINTER(RowmaxCountParams), _vp]),
    "lbfq_head_fp8_quant": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "lbfq_blasst_scan": (_i32, [_vp, _vp, _i64, _i64, _i64, _f32, _vp, _vp, _vp, _vp]),
    "lbfq_blasst_keep": (_i32, [_vp, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp]),
    "lbfq_blasst_attend": (_i32, [ctypes.POINTER(BlasstAttendParams), _vp]),
    "lbfq_sdpa_dequant": (_i32, [ctypes.POINTER(SdpaDequantParams), _vp]),
    "lbfq_sdpa_fwd": (_i32, [ctypes.POINTER(SdpaParams), _vp]),
    "lbfq_hbm_stream": (_i32, [_i32, _vp, _vp, _i64, _i32, _vp, _vp]),
    "lbfq_issue_probe": (_i32, [_i32, _i32, _i32, _vp, _vp, _vp]),
    "lbfq_selftest_cvt_fp8": (_i32, [_vp, _i64, _vp, _vp]),
    "lbfq_selftest_mfma": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp]),
}

EXPORTED = tuple(_SIGS)

_lib = None


class HipLibraryError(RuntimeError):
    pass


def load(require_gpu: bool = True):
    """Load the library (cached).  Raises if it is absent or no GPU is visible."""
    global _lib
    if require_gpu and not torch.cuda.is_available():
        raise HipLibraryError("low_bit_fake_quant needs a ROCm GPU: torch.cuda.is_available() is False")
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryError(
                f"{LIB_PATH} is missing; build it with `python low-bit-attention-fake-quant_amd/build_lib.py`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load(require_gpu=False).lbfq_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(msg or f"{what}: invalid argument")
        raise HipLibraryError(msg or f"{what}: failed with code {rc}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
