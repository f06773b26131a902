"""Wan2.1 call-site helpers: sequence padding and synthetic Wan-shaped inputs.

``pad_qkv`` follows the reference Wan hook (``bench/wan_attention_hook.py:
249-294``): S is padded to the LCM of the block sizes the quantisers and the
attention need, Q with zero rows and K/V by repeating their last row (padded
keys are attended, not masked); the caller slices the output back to S.

``make_inputs`` builds the benchmark workloads (B=1, bf16, NHD) on the CPU
from ``torch.Generator().manual_seed(seed)`` so the GPU and the CPU oracle
see identical bits:

* K ~ N(0,1) + per-(head, channel) bias ~ N(0, sigma=2); D/16 outlier
  channels (chosen by a seeded randperm per head) have their whole channel
  scaled by 10;
* Q, V ~ N(0,1); ``q_clusters``: Q = one of C centroids ~ N(0,1)^D (uniform
  assignment) + N(0, 0.3) noise; ``v_bias``: V += per-channel bias ~ N(0,1);
* ``field``: Q and K += a shared smooth field over the (t, h, w) latent grid
  (a few low-wavenumber Fourier modes), which makes attention spatially
  local.
"""

from __future__ import annotations

import functools
import math
from dataclasses import dataclass

import torch

from .config import QuantConfig


def pad_length(s: int, cfg: QuantConfig) -> int:
    sizes = [cfg.fp8_block_size, cfg.v_fp8_block_size, cfg.p_requant_block_m, cfg.p_requant_block_n]
    if cfg.smoothing == "full":
        sizes.append(cfg.q_smooth_block_size)
    if cfg.v_smooth_mode == "per_block":
        sizes.append(cfg.v_smooth_block_size)
    lcm = functools.reduce(lambda a, b: a * b // math.gcd(a, b), sizes, 1)
    return s + (lcm - s % lcm) % lcm


def pad_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cfg: QuantConfig):
    """Pad (B,S,H,D) tensors to the block LCM; returns (q, k, v, original S)."""
    b, s, h, d = q.shape
    sp = pad_length(s, cfg)
    pad = sp - s
    if pad == 0:
        return q, k, v, s
    qp = torch.cat([q, q.new_zeros(b, pad, h, d)], dim=1)
    kp = torch.cat([k, k[:, -1:].expand(b, pad, h, d)], dim=1)
    vp = torch.cat([v, v[:, -1:].expand(b, pad, h, d)], dim=1)
    return qp, kp, vp, s


@dataclass(frozen=True)
class Workload:
    name: str
    H: int
    N: int
    D: int
    cfg: QuantConfig
    q_clusters: int = 0
    v_bias: bool = False
    field_grid: tuple | None = None


def workloads() -> dict:
    """The five BASELINE configurations (index 0..4)."""
    c0 = QuantConfig(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="off",
                     q_kmeans_k=None, p_requant=False)
    c1 = QuantConfig(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="k_only",
                     q_kmeans_k=None, p_requant=True, p_quant="elementwise", rowmax_mode="online",
                     p_requant_block_m=64, p_requant_block_n=64)
    c2 = QuantConfig(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="full",
                     q_smooth_block_size=256, q_kmeans_k=32, p_requant=True, p_quant="dynamic",
                     rowmax_mode="qm_k", p_requant_block_m=64, p_requant_block_n=64)
    c3 = QuantConfig(qk_quant="mxfp8", mxfp8_block_size=32, qk_hadamard=True, v_quant="mxfp8",
                     v_mxfp8_block_size=64, v_kmeans_k=64, v_smooth_mode="per_block", v_smooth_block_size=64,
                     smoothing="full", q_kmeans_k=32, p_requant=True, p_quant="mx", rowmax_mode="online",
                     p_requant_block_m=64, p_requant_block_n=64)
    # lambda frozen once by calibrate_blasst_lambda on the full 40-head x 75600
    # workload (seed 0): 50.0% of the (row, K-block) decisions skip
    c4 = QuantConfig(qk_quant="fp8_block", fp8_block_size=64, v_quant="fp8_channel", smoothing="full",
                     q_smooth_block_size=256, q_kmeans_k=32, p_requant=True, p_quant="dynamic",
                     rowmax_mode="qm_k", p_requant_block_m=64, p_requant_block_n=64, blasst_lambda=1.59e-9,
                     blasst_fill="mean_a1.5")
    return {
        0: Workload("plumbing_h2_n1024_d64", 2, 1024, 64, c0),
        1: Workload("wan1.3b_h12_n32760_d128", 12, 32760, 128, c1),
        2: Workload("wan14b_h40_n32760_d128_dynP_qmk", 40, 32760, 128, c2, q_clusters=32),
        3: Workload("wan14b_h40_n32760_d128_mxfp8", 40, 32760, 128, c3, q_clusters=32, v_bias=True),
        4: Workload("wan14b720p_h40_n75600_d128_blasst", 40, 75600, 128, c4, q_clusters=0,
                    field_grid=(21, 45, 80)),
    }


def _field(grid, h: int, d: int, gen: torch.Generator, modes: int = 6, amp: float = 2.0) -> torch.Tensor:
    """Smooth low-frequency field over the (t, h, w) grid, (N, H, D) fp32."""
    T, Hh, W = grid
    t = torch.arange(T, dtype=torch.float32).view(T, 1, 1)
    y = torch.arange(Hh, dtype=torch.float32).view(1, Hh, 1)
    x = torch.arange(W, dtype=torch.float32).view(1, 1, W)
    out = torch.zeros(T * Hh * W, h, d)
    for _ in range(modes):
        kt, ky, kx = (torch.randint(0, 3, (3,), generator=gen).float() * torch.rand(3, generator=gen))
        ph = torch.rand(1, generator=gen).item() * 2 * math.pi
        wave = torch.cos(2 * math.pi * (kt * t / T + ky * y / Hh + kx * x / W) + ph).reshape(-1, 1, 1)
        coef = torch.randn(1, h, d, generator=gen)
        out += wave * coef
    return out * (amp / math.sqrt(modes))


def make_inputs(w: Workload, *, seed: int = 0, heads: int | None = None, dtype=torch.bfloat16):
    """CPU (q, k, v) of shape (1, N, H, D) for workload ``w`` (unpadded)."""
    h = heads or w.H
    n, d = w.N, w.D
    gen = torch.Generator().manual_seed(seed)
    n_out = max(1, d // 16)
    if w.q_clusters:
        cent = torch.randn(h, w.q_clusters, d, generator=gen)
        assign = torch.randint(0, w.q_clusters, (n, h), generator=gen)
        q = torch.gather(cent.unsqueeze(0).expand(n, h, w.q_clusters, d), 2,
                         assign.view(n, h, 1, 1).expand(n, h, 1, d)).squeeze(2)
        q = q + 0.3 * torch.randn(n, h, d, generator=gen)
    else:
        q = torch.randn(n, h, d, generator=gen)
    k = torch.randn(n, h, d, generator=gen) + 2.0 * torch.randn(1, h, d, generator=gen)
    scale = torch.ones(1, h, d)
    for hh in range(h):
        idx = torch.randperm(d, generator=gen)[:n_out]
        scale[0, hh, idx] = 10.0
    k = k * scale
    v = torch.randn(n, h, d, generator=gen)
    if w.v_bias:
        v = v + torch.randn(1, h, d, generator=gen)
    if w.field_grid is not None:
        f = _field(w.field_grid, h, d, gen)
        q = q + f
        k = k + f
    return tuple(t.unsqueeze(0).to(dtype).contiguous() for t in (q, k, v))


def blasst_skip_rate(q, k, v, cfg, lam: float) -> float:
    """Fraction of (row, K-block) decisions BLASST skips at lambda ``lam``:
    stats[..., 0].sum() / stats[..., 1].sum() (attention_triton.py:404-407),
    for (B,S,H,D) device tensors already padded to the block LCM."""
    import dataclasses

    from .attention import _lazy_preprocess, quantize_operands
    from .attention_kernel import launch_attention
    sm = q.shape[-1] ** -0.5
    c = dataclasses.replace(cfg, blasst_lambda=float(lam))
    ops = quantize_operands(_lazy_preprocess(q, k, v, c), c, sm)
    _, stats = launch_attention(ops, c, sm, q.dtype, return_blasst_stats=True)
    st = stats.sum(dim=(0, 1))
    return (st[0] / st[1]).item()


def calibrate_blasst_lambda(q, k, v, cfg, target: float = 0.5, iters: int = 24) -> tuple[float, float]:
    """Bisection on log(lambda) for the skip rate ``target`` (the skip rate
    grows with lambda).  Returns (lambda, measured skip rate)."""
    lo, hi = math.log(1e-12), math.log(0.999)
    best = (math.exp(hi), blasst_skip_rate(q, k, v, cfg, math.exp(hi)))
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        r = blasst_skip_rate(q, k, v, cfg, math.exp(mid))
        if abs(r - target) < abs(best[1] - target):
            best = (math.exp(mid), r)
        if r > target:
            hi = mid
        else:
            lo = mid
    return best


def _main(argv=None) -> int:
    import argparse
    import json
    import sys
    ap = argparse.ArgumentParser(description="Calibrate BLASST lambda of a Wan workload on the GPU")
    ap.add_argument("--config", type=int, default=4)
    ap.add_argument("--target", type=float, default=0.5)
    ap.add_argument("--heads", type=int, default=0)
    args = ap.parse_args(argv)
    w = workloads()[args.config]
    q, k, v = make_inputs(w, seed=0, heads=args.heads or None)
    q, k, v, _ = pad_qkv(q, k, v, w.cfg)
    dev = torch.device("cuda:0")
    lam, rate = calibrate_blasst_lambda(q.to(dev), k.to(dev), v.to(dev), w.cfg, target=args.target)
    print(json.dumps({"config": args.config, "workload": w.name, "heads": q.shape[2], "lambda": lam,
                      "skip_rate": rate, "target": args.target}))
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    raise SystemExit(_main())
