"""Pins the end-to-end oracle pipeline (reference attention.py:166-321, 505-806)
by invariances that hold whatever the quantisers do:

* Q k-means reorder with per-row MX Q/K scales and no Q smoothing only permutes
  independent query rows, so with the inverse gather the output equals the
  output without reorder bit for bit;
* V k-means with the K co-permutation permutes keys; with per-channel V scales,
  per-row MX K scales, a permutation-invariant K mean and a fixed qm_k row max
  (elementwise P), every P code is unchanged, so only the fp32 summation order
  of the output changes;
* the SDPA path (p_requant=False) equals torch's CPU SDPA on the dequantised
  tensors.
"""

import dataclasses
import math

import torch
import torch.nn.functional as F

from conftest import cpu_randn
from oracle import pipeline as opipe


@dataclasses.dataclass(frozen=True)
class Cfg:
    qk_quant: str = "mxfp8"
    fp8_block_size: int = 64
    mxfp8_block_size: int = 32
    qk_hadamard: bool = False
    qk_hadamard_random_sign: bool = True
    qk_hadamard_seed: int = 0
    v_quant: str = "fp8_channel"
    v_fp8_block_size: int = 64
    v_mxfp8_block_size: int = 64
    smoothing: str = "off"
    q_smooth_block_size: int = 256
    q_kmeans_k: int | None = None
    q_kmeans_iters: int = 3
    q_kmeans_seed: int = 0
    v_kmeans_k: int | None = None
    v_kmeans_iters: int = 3
    v_kmeans_seed: int = 0
    v_smooth_mode: str = "off"
    v_smooth_block_size: int = 64
    p_requant: bool = True
    p_quant: str = "elementwise"
    p_max_offset: int = 8
    p_mx_block_n: int = 0
    p_requant_block_m: int = 64
    p_requant_block_n: int = 64
    rowmax_mode: str = "online"
    blasst_lambda: float | None = None
    blasst_fill: str = "zero"
    blasst_fill_alpha: float = 1.0
    blasst_uta_bins: int = 16


def _qkv(s=512, h=2, d=64, seed=0):
    q = cpu_randn(1, s, h, d, seed=seed)
    k = cpu_randn(1, s, h, d, seed=seed + 1)
    v = cpu_randn(1, s, h, d, seed=seed + 2)
    return q, k, v


def test_q_reorder_with_inverse_gather_is_row_permutation_invariant():
    q, k, v = _qkv(seed=3)
    base = opipe.fake_quant_attention(q, k, v, Cfg(p_quant="dynamic"))
    reo = opipe.fake_quant_attention(q, k, v, Cfg(p_quant="dynamic", q_kmeans_k=8))
    assert torch.equal(base, reo)


def test_v_kmeans_copermutation_keeps_output_with_fixed_rowmax():
    q, k, v = _qkv(seed=5)
    cfg = Cfg(smoothing="full", q_smooth_block_size=128, rowmax_mode="qm_k", p_quant="elementwise")
    base = opipe.fake_quant_attention(q, k, v, cfg)
    perm = opipe.fake_quant_attention(q, k, v, dataclasses.replace(cfg, v_kmeans_k=8))
    assert (base.float() - perm.float()).abs().max().item() <= 2 ** -7 * base.float().abs().max().item()
    assert torch.nn.functional.cosine_similarity(base.float().flatten(), perm.float().flatten(), dim=0) > 0.99999


def test_sdpa_path_equals_torch_sdpa_on_dequantised_tensors():
    q, k, v = _qkv(seed=7)
    cfg = Cfg(qk_quant="fp8_block", p_requant=False)
    out = opipe.fake_quant_attention(q, k, v, cfg)
    qc, qs, qmeta = opipe.quant_qk(q, cfg)
    kc, ks, kmeta = opipe.quant_qk(k, cfg)
    vc, vs, vmeta = opipe.quant_v(v, cfg)
    qd = opipe.dequant_qk(qc, qs, qmeta, torch.bfloat16).permute(0, 2, 1, 3).float()
    kd = opipe.dequant_qk(kc, ks, kmeta, torch.bfloat16).permute(0, 2, 1, 3).float()
    vd = opipe.dequant_v(vc, vs, vmeta, torch.bfloat16).permute(0, 2, 1, 3).float()
    ref = F.scaled_dot_product_attention(qd, kd, vd, scale=1.0 / math.sqrt(64)).permute(0, 2, 1, 3)
    assert (out.float() - ref).abs().max().item() <= 1e-2
    assert torch.nn.functional.cosine_similarity(out.float().flatten(), ref.flatten(), dim=0) > 0.9999
