#!/usr/bin/env python3
"""Benchmark of the MI355X fake-quant attention hot path.

Workload (default ``--config 2``): Wan2.1-14B-shaped self-attention, B=1,
H=40, N=32760 (padded to 32768 per the Wan hook), D=128, bf16, Q/K
fp8_block 64, V fp8_channel, full smoothing (q_smooth 256), Q k-means 32,
dynamic P with the qm_k row-max estimate.  Synthetic inputs (seeded CPU
generator), no checkpoint.

One *step* = one launch of the FP8-MFMA attention kernel over the resident
quantised operands (the reference times fake_quant_attention with the
preprocess cached).  ``value`` = 4*N^2*D*H / step time in TFLOP/s (unpadded
N).  The prepass kernels (quantisers, qm.K_s, k-means) are timed separately
and reported in GB/s; the whole fake_quant_attention call with cached
preprocess is reported as ``e2e_cached``.  ``cpu_baseline`` times the CPU
oracle's attention on one head and a bounded row sample; the same sample
gives the error of the GPU output against the oracle at full size, both
against the reference (its own bf16-dequant scores) and against the
reference algorithm replayed on the kernel's scores.  With the default
config the attention of BASELINE configs 1, 3 and 4 is timed in the same run
(``other_configs``; config 4's BLASST skip rate included).
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "low-bit-attention-fake-quant_amd")
for _p in (REPO, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

FP8_PEAK_TFLOPS = 5000.0   # MI355X dense FP8 MFMA (datasheet)
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3   # MI355X fp32 (vector / MFMA, dense)
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (datasheet)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _events_time(fn, iters: int, warmup: int) -> float:
    """Average ms per call of fn() measured with HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def cpu_info():
    """The host CPU the baseline runs on and the threads it may use: the
    model name, the logical CPU count, the CPUs this process may run on
    (affinity) and the cgroup CPU quota where one is set; threads = the
    affinity count, capped by the quota."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    logical = os.cpu_count()
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = logical
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q_, per = f.read().split()[:2]
            if q_ != "max":
                quota = int(q_) / int(per)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    return {"model": model, "logical_cpus": logical, "affinity_cpus": affinity, "cgroup_cpu_quota": quota}, threads


def _sample_rows(order, n_real, rows_sample, seed=1):
    gen = torch.Generator().manual_seed(seed)
    cand = torch.nonzero(order < n_real).flatten()
    return cand[torch.randperm(len(cand), generator=gen)[:rows_sample]].sort().values


def _err(got, want):
    d = (got - want).abs()
    ulp = torch.pow(2.0, torch.floor(torch.log2(want.abs().clamp_min(2.0 ** -126))) - 7)
    g64, w64 = got.double().flatten(), want.double().flatten()
    cos = ((g64 @ w64) / (g64.norm() * w64.norm()).clamp_min(1e-300)).item()
    return {"cos": cos, "max_abs": d.max().item(), "max_abs_beyond_1_bf16_ulp": (d - ulp).clamp_min(0).max().item(),
            "frac_gt_1e-2": (d > 1e-2).float().mean().item()}


def oracle_error(q, k, v, cfg, out_gpu, n_real, rows_sample, sm_scale):
    """Part of the cpu_baseline / error legs (the oracle as checker): the CPU
    oracle of the reference path on head 0 -- preprocess (untimed), then the
    P-requant path (quantise the head, row-max estimate, streaming attention)
    for a bounded sample of real query rows -- against the GPU output at full
    size.  Also the oracle with exact (fp32) dequantised Q/K: the reference's
    own sensitivity to its bf16 rounding of the dequantised Q/K
    (attention.py:532-535), the bound the tests hold the kernel to.  Returns
    (error dict, seconds of the timed reference pass, rows, S)."""
    from oracle import pipeline as opipe
    q0, k0, v0 = (t[:, :, :1].contiguous() for t in (q, k, v))
    s = q0.shape[1]
    t0 = time.time()
    qw, kw, vw, qm, v_alpha, q_km, _ = opipe.preprocess(q0, k0, v0, cfg)
    prep_s = time.time() - t0
    order = q_km["order"][0] if q_km is not None else torch.arange(s)
    rows = _sample_rows(order, n_real, rows_sample)
    t1 = time.time()
    o = opipe.p_requant_path(qw, kw, vw, qm, v_alpha, cfg, sm_scale, torch.bfloat16, rows=rows)
    attn_s = time.time() - t1
    o32 = opipe.p_requant_path(qw, kw, vw, qm, v_alpha, cfg, sm_scale, torch.bfloat16, rows=rows,
                               qk_dequant_dtype=torch.float32)
    gpu_rows = out_gpu[0, order[rows], 0].float().cpu()
    ref_rows, ref32_rows = o[0, :, 0].float(), o32[0, :, 0].float()
    fin = torch.isfinite(ref_rows) & torch.isfinite(ref32_rows) & torch.isfinite(gpu_rows)
    err = _err(gpu_rows[fin], ref_rows[fin])
    own = _err(ref32_rows[fin], ref_rows[fin])
    err.update({"rows": len(rows), "head": 0, "rows_fraction_of_head": len(rows) / n_real,
                "vs": "CPU oracle of the reference path (its bf16-dequant scores; not SDPA)",
                "vs_exact_dequant_reference": _err(gpu_rows[fin], ref32_rows[fin]),
                "reference_own_gap": {"cos": own["cos"], "max_abs": own["max_abs"],
                                      "note": "reference with fp32- vs bf16-dequantised Q/K on the same rows"},
                "nonfinite_rows_left_out": int((~fin).any(-1).sum()), "oracle_preprocess_s": prep_s})
    return err, attn_s, len(rows), s


def cpu_baseline_and_error(q, k, v, cfg, out_gpu, n_real, rows_sample, sm_scale):
    """The CPU baseline: the oracle's P-requant pass on head 0 for a bounded row
    sample, timed on the host's cores (the reference's timing likewise includes
    quant/dequant and excludes the cached preprocess, bench/eval_wan21.py:
    208-255); the same sample gives the error against the reference.  Returns
    (cpu_baseline dict, error dict, error against the replay on the kernel's
    scores)."""
    info, threads = cpu_info()
    torch.set_num_threads(threads)
    err, attn_s, nrows, s = oracle_error(q, k, v, cfg, out_gpu, n_real, rows_sample, sm_scale)
    d, h = q.shape[-1], q.shape[2]
    flops = 4.0 * nrows * s * d
    cpu = {"value": flops / attn_s / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "cpu": info,
           "sample": f"oracle P-requant path (quantise head 0, row-max estimate, streaming attention) for "
                     f"{nrows} of {n_real} query rows ({100 * nrows / n_real:.1f}%) x {s} keys of 1 of {h} heads "
                     f"({100 * nrows / n_real / h:.2f}% of the workload's rows), D={d}, fp32 torch on {threads} "
                     f"threads of {info['model']} ({attn_s:.1f} s; the head's preprocess, "
                     f"{err['oracle_preprocess_s']:.1f} s, not timed)",
           "workload_fraction": nrows / n_real / h, "seconds": attn_s}
    log("error against the replay on the kernel's scores ...")
    err_replay = replay_error(q, k, v, cfg, sm_scale, out_gpu, n_real, min(rows_sample, 2048))
    return cpu, err, err_replay


def replay_error(q, k, v, cfg, sm_scale, out_gpu, n_real, rows_sample):
    """Part of the cpu_baseline leg (the oracle as checker): the GPU output
    against the oracle's reference algorithm replayed on the kernel's own
    scores (tests/parity.py), for head 0 and a row sample -- the strict part of
    the parity check at full size (untimed)."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import parity
    from oracle import pipeline as opipe
    q0, k0, v0 = (t[:, :, :1].contiguous() for t in (q, k, v))
    ops0, _ = parity.kernel_operands(q0, k0, v0, cfg, torch.device("cuda:0"), sm_scale)
    qw, kw, vw, qm, v_alpha, q_km, _ = opipe.preprocess(q0, k0, v0, cfg)
    order = q_km["order"][0] if q_km is not None else torch.arange(q0.shape[1])
    rows = _sample_rows(order, n_real, rows_sample)
    u = parity.kernel_scores(ops0, cfg, sm_scale, rows=rows.to(torch.int32))
    rm = ops0.rowmax.cpu() if ops0.rowmax is not None else None
    rep, dbg = opipe.p_requant_path(qw, kw, vw, qm, v_alpha, cfg, sm_scale, torch.float32, rows=rows,
                                    scores_log2=u, rowmax_log2=rm, return_debug=True)
    got = out_gpu[0, order[rows], 0].float().cpu()
    want = rep[0, :, 0].float()
    d = (got - want).abs()
    tol = parity.tolerance(want) + dbg["flip_allowance"][0, 0].float()
    return {"cos": parity.cosine(got, want), "max_abs": d.max().item(),
            "elements_beyond_tolerance": int((d > tol).sum()), "rows": len(rows), "head": 0,
            "vs": "the reference algorithm replayed on the kernel's own scores (strict parity)"}


def prepass_bytes(ops, in_bytes: int) -> int:
    """Algorithmic bytes of the prepass: the caller's Q/K/V read once plus every
    tensor the attention kernel reads written once (codes with their padding
    rows, scales, the qm correction table, row-max estimates, V block means,
    V tile column sums, the Q row map)."""
    out = 0
    for name in ("q_codes", "q_scale", "k_codes", "k_scale", "v_codes_t", "v_scale", "bias", "rowmax", "v_alpha",
                 "out_row_map", "v_colsum"):
        t = getattr(ops, name, None)
        if t is not None:
            out += t.numel() * t.element_size()
    return in_bytes + out


def other_configs(configs, dev, steps: int = 5, err_rows: int = 1024):
    """The other BASELINE configs in the same run: attention time (inputs,
    preprocess and quantisation untimed), the prepass (quantisers + qm.K_s)
    and the cached end-to-end call, and the error against the oracle on a row
    sample of head 0.  Config 4 adds its BLASST skip rate, the wave-tile skip
    fractions, the fraction of the dense schedule's MFMAs it issues, the
    uta16 fill and the dense kernel on the same shape."""
    from low_bit_fake_quant import fake_quant_attention, prepare_for_attention
    from low_bit_fake_quant.attention import _lazy_preprocess, quantize_operands
    from low_bit_fake_quant.attention_kernel import attention_flops, launch_attention
    from low_bit_fake_quant.wan import make_inputs, pad_qkv, workloads
    res = {}
    for c in configs:
        w = workloads()[c]
        cfg = w.cfg
        q, k, v = make_inputs(w, seed=0)
        q, k, v, n = pad_qkv(q, k, v, cfg)
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        sm = 1.0 / (w.D ** 0.5)
        prep = _lazy_preprocess(qd, kd, vd, cfg)
        q_ms = _events_time(lambda: quantize_operands(prep, cfg, sm), 10, 2)
        ops = quantize_operands(prep, cfg, sm)
        pb = prepass_bytes(ops, 3 * qd.numel() * qd.element_size())
        ref_bytes = 3 * qd.numel() * (qd.element_size() + 1)
        ms = _events_time(lambda: launch_attention(ops, cfg, sm, torch.bfloat16), steps, 3)
        fl = attention_flops(n, w.H, w.D)
        r = {"workload": w.name, "ms": ms, "TFLOPs": fl / (ms * 1e-3) / 1e12,
             "frac_of_fp8_peak": fl / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS,
             "prepass": {"quantise_qmk_ms": q_ms, "algorithmic_bytes": pb,
                         "GBps": pb / (q_ms * 1e-3) / 1e9, "frac_of_hbm_peak": pb / (q_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "reference_bytes_GBps": ref_bytes / (q_ms * 1e-3) / 1e9}}
        cache = prepare_for_attention(qd, kd, vd, cfg)
        r["e2e_cached_ms"] = _events_time(lambda: fake_quant_attention(qd, kd, vd, cfg, preprocess_cache=cache), 3, 1)
        r["e2e_cached_TFLOPs"] = fl / (r["e2e_cached_ms"] * 1e-3) / 1e12
        del cache, prep
        if cfg.blasst_lambda is not None:
            _, stats, wt = launch_attention(ops, cfg, sm, torch.bfloat16, return_blasst_stats=True,
                                            return_wave_tiles=True)
            st = stats.sum(dim=(0, 1))
            nt = -(-n // cfg.p_requant_block_n)   # decision blocks per row
            wave_tiles = wt.shape[0] * wt.shape[1] * nt
            w_all = wt[..., 0].sum().item() / wave_tiles
            # a (wave, tile) that every row skips issues its 4 QK MFMAs but not its 4
            # PV MFMAs (fill x V column sums instead) when the column-sum table exists
            elide = ops.v_colsum is not None
            r.update({"blasst_lambda": cfg.blasst_lambda, "blasst_fill": cfg.blasst_fill,
                      "skip_rate": (st[0] / st[1]).item(), "TFLOPs_note": "dense-equivalent (4 N^2 D H)",
                      # (wave of 32 rows, 64-key tile) pairs: every row skipped (the softmax is
                      # elided) / some row skipped
                      "wave_tiles_all_skipped": w_all,
                      "wave_tiles_some_skipped": wt[..., 1].sum().item() / wave_tiles,
                      "mfma_executed_fraction": 1.0 - 0.5 * w_all if elide else 1.0,
                      "mfma_executed_note": "of the dense schedule's 8 MFMAs per wave and tile, from the "
                                            "kernel's wave-tile counters (rocprof SQ_INSTS_VALU_MFMA_MOPS_F8 / 256 agrees)"})
            cd = dataclasses.replace(cfg, blasst_lambda=None)
            ms_d = _events_time(lambda: launch_attention(ops, cd, sm, torch.bfloat16), steps, 3)
            r["dense_same_shape"] = {"ms": ms_d, "TFLOPs": fl / (ms_d * 1e-3) / 1e12,
                                     "blasst_speedup_vs_dense": ms_d / ms,
                                     "note": "the same operands and kernel family with BLASST off, same run"}
            log(f"config {c} dense (BLASST off): {ms_d:.3f} ms/launch")
            if cfg.blasst_fill == "mean_a1.5":  # the second fill BASELINE names (same decisions)
                cu = dataclasses.replace(cfg, blasst_fill="uta16_a1.5")
                ms_u = _events_time(lambda: launch_attention(ops, cu, sm, torch.bfloat16), steps, 3)
                r["uta16_a1.5"] = {"ms": ms_u, "TFLOPs": fl / (ms_u * 1e-3) / 1e12,
                                   "blasst_speedup_vs_dense": ms_d / ms_u, "mfma_executed_fraction": 1.0}
                log(f"config {c} uta16_a1.5: {ms_u:.3f} ms/launch")
        log(f"config {c}: {ms:.3f} ms/launch, {r['TFLOPs']:.1f} TFLOP/s; prepass {q_ms:.3f} ms")
        out = launch_attention(ops, cfg, sm, torch.bfloat16)
        del ops, qd, kd, vd
        torch.cuda.empty_cache()
        if err_rows:
            try:
                r["err_vs_oracle"], _, _, _ = oracle_error(q, k, v, cfg, out, n, err_rows, sm)
            except Exception as e:  # report, do not lose the timings
                r["err_vs_oracle"] = {"error": repr(e)}
            log(f"config {c}: err vs oracle {r['err_vs_oracle']}")
        res[str(c)] = r
        del out, q, k, v
        torch.cuda.empty_cache()
    return res


def path_a(dev, steps: int = 5):
    """The reference's path A (``p_requant=False``) on its native kernels: config
    0 end to end (timed, and its whole output against the oracle), and the
    attention kernel alone at config 1's shape with P not quantised (dense-
    equivalent 4 N^2 D H flops against the bf16 MFMA peak)."""
    from low_bit_fake_quant import fake_quant_attention
    from low_bit_fake_quant.attention import _lazy_preprocess, launch_sdpa, sdpa_operands
    from low_bit_fake_quant.wan import make_inputs, pad_qkv, workloads
    res = {}
    w = workloads()[0]
    q, k, v = make_inputs(w, seed=0)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    ms0 = _events_time(lambda: fake_quant_attention(qd, kd, vd, w.cfg), 20, 3)
    out = fake_quant_attention(qd, kd, vd, w.cfg).cpu()
    r0 = {"workload": w.name, "e2e_ms": ms0}
    # the same call captured once in a HIP graph and replayed (its ~10 launches
    # are the cost at this size); the replay must equal the eager output
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            gout = fake_quant_attention(qd, kd, vd, w.cfg)
        r0["e2e_graph_ms"] = _events_time(g.replay, 20, 3)
        r0["graph_equals_eager"] = bool(torch.equal(gout.cpu(), out))
    except Exception as e:  # report, do not lose the rest of the bench line
        r0["e2e_graph_ms"], r0["graph_equals_eager"] = None, repr(e)
    try:
        from oracle import pipeline as opipe
        r0["err_vs_oracle"] = _err(out, opipe.fake_quant_attention(q, k, v, w.cfg))
        r0["err_vs_oracle"]["rows"] = "all"
    except Exception as e:  # report, do not lose the timing
        r0["err_vs_oracle"] = {"error": repr(e)}
    res["config0"] = r0
    log(f"path A config 0: {ms0:.3f} ms ({r0['e2e_graph_ms']} ms as a graph replay, equal to eager: "
        f"{r0['graph_equals_eager']}), err {r0['err_vs_oracle']}")
    w1 = workloads()[1]
    cfg = dataclasses.replace(w1.cfg, p_requant=False)
    q, k, v = make_inputs(w1, seed=0)
    q, k, v, n = pad_qkv(q, k, v, cfg)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    sm = 1.0 / (w1.D ** 0.5)
    prep = _lazy_preprocess(qd, kd, vd, cfg)
    ops_ms = _events_time(lambda: sdpa_operands(prep, cfg, sm, torch.bfloat16), steps, 1)
    sops = sdpa_operands(prep, cfg, sm, torch.bfloat16)
    ms = _events_time(lambda: launch_sdpa(sops, sm, torch.bfloat16), steps, 1)
    fl = 4.0 * n * n * w1.D * w1.H
    res["config1_shape"] = {"workload": w1.name + " with p_requant=False", "attention_ms": ms,
                            "quantise_dequantise_ms": ops_ms, "TFLOPs": fl / (ms * 1e-3) / 1e12,
                            "frac_of_bf16_peak": fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                            "note": "bf16 MFMA, P unquantised (two PV products: P's bf16 rounding and residual)"}
    log(f"path A at config 1's shape: {ms:.3f} ms, {res['config1_shape']['TFLOPs']:.1f} TFLOP/s")
    del sops, prep, qd, kd, vd
    torch.cuda.empty_cache()
    return res


def hbm_ceiling(dev, nbytes: int = 1 << 31, grids=(1024, 2048, 4096, 8192)):
    """The HBM ceiling measured with this library's own streaming kernels
    (lbfq_hbm_stream, global_load/store_dwordx4): read-only, write-only and
    copy over `nbytes` (2 GiB, far beyond the 256 MB MALL), the best of a few
    grid sizes each; GB/s counts the bytes moved (copy: read + write)."""
    from low_bit_fake_quant import _lib
    lib = _lib.load()
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    st = _lib.stream_handle(dev)
    res = {}
    for mode, name, mult in ((0, "read", 1), (1, "write", 1), (2, "copy", 2)):
        best = None
        for g in grids:
            def fn(mode=mode, g=g):
                _lib.check(lib.lbfq_hbm_stream(mode, src.data_ptr(), dst.data_ptr(), nbytes, g, sink.data_ptr(), st),
                           "lbfq_hbm_stream")
            ms = _events_time(fn, 5, 2)
            gbs = mult * nbytes / (ms * 1e-3) / 1e9
            if best is None or gbs > best[0]:
                best = (gbs, g, ms)
        res[name] = {"GBps": best[0], "grid": best[1], "ms": best[2]}
        log(f"hbm stream {name}: {best[0]:.0f} GB/s (grid {best[1]})")
    del src, dst
    torch.cuda.empty_cache()
    return res


ISSUE_OPS = ("v_mul_f32", "v_add_f32", "v_fma_f32", "v_max3_f32", "v_exp_f32", "v_cvt_pk_fp8_f32",
             "v_permlane32_swap", "mfma_f32_32x32x64_f8", "tile_mix", "tile_mix_valu_only")


def issue_costs(dev, iters: int = 2000):
    """lbfq_issue_probe on one CU: cycles per wave-instruction at the SIMD for
    each instruction class the attention step is made of, and cycles per
    wave-tile of the step's inherent mix (8 MFMAs + 198 VALU, all independent:
    a perfect schedule), at 1 and 2 waves per SIMD (the attention kernel runs
    2).  Per SIMD: (latest end - earliest start of its waves) / (waves x
    iterations x instructions per iteration)."""
    from low_bit_fake_quant import _lib
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    sink = torch.zeros(512, dtype=torch.float32, device=dev)
    rec = torch.zeros(8 * 3, dtype=torch.int64, device=dev)
    per_iter = [16] * 7 + [8, 1, 1]
    out = {}
    for w in (1, 2):
        row = {}
        for op, name in enumerate(ISSUE_OPS):
            _lib.check(lib.lbfq_issue_probe(op, w, iters, rec.data_ptr(), sink.data_ptr(), st), "lbfq_issue_probe")
            torch.cuda.synchronize()
            r = rec[:3 * 4 * w].view(4 * w, 3).cpu().tolist()
            worst = 0.0
            for simd in range(4):
                ws = [x for x in r if x[2] == simd]
                if len(ws) == w:
                    span = max(x[1] for x in ws) - min(x[0] for x in ws)
                    worst = max(worst, span / (w * iters * per_iter[op]))
            row[name] = worst
        out[f"{w}_wave_per_simd"] = row
        log(f"issue costs at {w} wave(s)/SIMD: " + ", ".join(f"{k} {v:.2f}" for k, v in row.items()))
    return out


def traffic_from_profile(config: int):
    """HBM bytes per attention launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, calibrated by a copy of known size), or None."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(REPO, "profiles", f"traffic_attn_fwd_c{config}_*.md"))):
        with open(path) as f:
            m = re.search(r"^hbm_bytes_per_launch:\s*(\d+)", f.read(), flags=re.M)
        if m:
            return int(m.group(1))
    return None


def clock_sample(ops, cfg, sm_scale, launches, flops, launch_attention, quiet=False):
    """Shader clock under a long run of the attention kernel: rocm-smi is
    sampled from a thread while `launches` launches run back to back.  The
    datasheet FP8 peak (5.0 PFLOP/s) is quoted at 2.4 GHz; the rate is also
    reported against that peak scaled to the median sampled clock."""
    import re
    import subprocess
    import threading

    def sclk_mhz():
        try:
            r = subprocess.run(["rocm-smi", "--showclocks", "--csv"], capture_output=True, text=True, timeout=10)
        except (OSError, subprocess.SubprocessError):
            return None
        m = re.search(r"card0,\((\d+)Mhz\),\d+,\((\d+)Mhz\)", r.stdout)
        return (int(m.group(2)), int(m.group(1))) if m else None

    launch_attention(ops, cfg, sm_scale, torch.bfloat16)
    torch.cuda.synchronize()
    idle = sclk_mhz()
    samples, stop = [], threading.Event()

    def sampler():
        t0 = time.time()
        while not stop.is_set():
            c = sclk_mhz()
            if c:
                samples.append((time.time() - t0, c[0], c[1]))
            time.sleep(0.25)

    th = threading.Thread(target=sampler)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    th.start()
    e0.record()
    for _ in range(launches):
        launch_attention(ops, cfg, sm_scale, torch.bfloat16)
    e1.record()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    ms = e0.elapsed_time(e1) / launches
    busy = [c for t, c, _ in samples[2:-2]] or [c for _, c, _ in samples]
    busy.sort()
    med = busy[len(busy) // 2] if busy else float("nan")
    tflops = flops / (ms * 1e-3) / 1e12
    peak_at_clk = FP8_PEAK_TFLOPS * med / 2400.0
    for t, c, mc in samples:
        log(f"t={t:5.2f}s sclk {c} MHz mclk {mc} MHz")
    res = {"launches": launches, "ms_per_launch": ms, "TFLOPs": tflops,
           "sclk_idle_MHz": idle[0] if idle else None, "sclk_median_MHz": med,
           "sclk_samples": len(samples), "frac_of_fp8_peak_2400MHz": tflops / FP8_PEAK_TFLOPS,
           "fp8_peak_at_median_clock_TFLOPs": peak_at_clk,
           "frac_of_clock_scaled_peak": tflops / peak_at_clk}
    if quiet:
        return res
    print(json.dumps(res))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--heads", type=int, default=0, help="override H (debug)")
    ap.add_argument("--cpu-rows", type=int, default=8192)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip timing configs 1, 3 and 4 beside the headline config")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="driver for rocprofv3 --pmc passes: a 1 GiB calibration copy, then one attention launch")
    ap.add_argument("--issue-floor", action="store_true",
                    help="issue costs of the attention step's instruction classes and of its inherent per-tile mix "
                         "(lbfq_issue_probe), the config's attention timed under a clock sample, and the floor they "
                         "imply; one JSON line")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only the HBM streaming probe (read / write / copy), one JSON line")
    ap.add_argument("--trace-timed-only", action="store_true",
                    help="for rocprofv3 --kernel-trace: the prepass, then only the warmup and timed attention "
                         "launches of the headline (no end-to-end, hook, diagnostic or other-config calls)")
    ap.add_argument("--path-a-only", action="store_true",
                    help="only the p_requant=False leg (config 0 end to end, the attention at config 1's shape); "
                         "one JSON line, for rocprofv3 --kernel-trace")
    ap.add_argument("--clock-sample", type=int, default=0, metavar="LAUNCHES",
                    help="run LAUNCHES attention launches back to back while sampling the shader clock with "
                         "rocm-smi; print the samples and the rate against the clock-scaled FP8 peak")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU per process; --gpus N>1 is not supported "
                          "(the path shards by heads with no communication)", "n_gpus": args.gpus}))
        return 2

    from low_bit_fake_quant import _lib, fake_quant_attention, prepare_for_attention
    from low_bit_fake_quant.attention import _lazy_preprocess, _prep_from_cache, quantize_operands
    from low_bit_fake_quant.attention_kernel import attention_flops, launch_attention
    from low_bit_fake_quant.wan import make_inputs, pad_qkv, workloads

    _lib.load()
    dev = torch.device("cuda:0")
    if args.hbm_ceiling:
        print(json.dumps({"hbm_stream": hbm_ceiling(dev), "bytes": 1 << 31}))
        return 0
    if args.path_a_only:
        print(json.dumps({"path_a": path_a(dev)}))
        return 0
    w = workloads()[args.config]
    cfg = w.cfg
    h = args.heads or w.H
    t0 = time.time()
    q, k, v = make_inputs(w, seed=0, heads=h)
    q, k, v, n_real = pad_qkv(q, k, v, cfg)
    log(f"inputs {tuple(q.shape)} generated in {time.time() - t0:.1f}s")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    b, s, _, d = qd.shape
    sm_scale = 1.0 / (d ** 0.5)

    # ---- prepass (preprocess + quantisation), timed per stage --------------
    res = {}
    torch.cuda.synchronize()
    prep_ms = _events_time(lambda: _lazy_preprocess(qd, kd, vd, cfg), 3, 1)
    prep = _lazy_preprocess(qd, kd, vd, cfg)
    quant_ms = _events_time(lambda: quantize_operands(prep, cfg, sm_scale), 20, 3)
    ops = quantize_operands(prep, cfg, sm_scale)
    torch.cuda.synchronize()
    log(f"prepass: preprocess {prep_ms:.3f} ms, quantise+qmk {quant_ms:.3f} ms")

    if args.pmc_pass:
        # a plain copy of known size (2^30 bytes read, 2^30 written) calibrates
        # FETCH_SIZE / WRITE_SIZE; then exactly one attention launch
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        launch_attention(ops, cfg, sm_scale, torch.bfloat16)
        torch.cuda.synchronize()
        log("pmc pass: calibration copy + one attention launch done")
        return 0

    if args.clock_sample:
        return clock_sample(ops, cfg, sm_scale, args.clock_sample, attention_flops(n_real, h, d, b), launch_attention)

    if args.issue_floor:
        costs = issue_costs(dev)
        props = torch.cuda.get_device_properties(dev)
        simds = props.multi_processor_count * 4
        # (wave of 32 queries, 64-key tile) pairs per SIMD: workgroups of 4 waves x 128 queries (eight-wave
        # workgroups of 256 queries launch as many waves wherever ceil(S / 256) = ceil(S / 128) / 2, as at S = 32760)
        wave_tiles = b * h * ((s + 127) // 128) * 4 * ((s + 63) // 64) / simds
        info = clock_sample(ops, cfg, sm_scale, 120, attention_flops(n_real, h, d, b), launch_attention,
                            quiet=True)
        mhz = info["sclk_median_MHz"]
        tile = costs["2_wave_per_simd"]["tile_mix"]
        floor_ms = tile * wave_tiles / (mhz * 1e3)
        kernel_cycles = info["ms_per_launch"] * 1e-3 * mhz * 1e6 / wave_tiles
        print(json.dumps({"issue_costs_cycles": costs, "simds": simds, "wave_tiles_per_simd": wave_tiles,
                          "sclk_median_MHz": mhz, "attention_ms": info["ms_per_launch"],
                          "attention_cycles_per_wave_tile": kernel_cycles,
                          "floor_cycles_per_wave_tile": tile, "floor_ms_at_sampled_clock": floor_ms,
                          "floor_ms_at_2400MHz": tile * wave_tiles / 2.4e6,
                          "floor_frac_of_fp8_peak_at_sampled_clock":
                              attention_flops(n_real, h, d, b) / (floor_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS,
                          "kernel_over_floor": kernel_cycles / tile}))
        return 0

    # ---- attention kernel: the timed step ----------------------------------
    out = launch_attention(ops, cfg, sm_scale, torch.bfloat16)
    torch.cuda.synchronize()
    ms = _events_time(lambda: launch_attention(ops, cfg, sm_scale, torch.bfloat16), args.steps, args.warmup)
    flops = attention_flops(n_real, h, d, b)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"attention: {ms:.3f} ms/launch, {tflops:.1f} TFLOP/s ({100 * tflops / FP8_PEAK_TFLOPS:.1f}% of FP8 peak)")
    if args.trace_timed_only:
        print(json.dumps({"config": args.config, "attention_launches": 1 + args.warmup + args.steps,
                          "timed_launches": args.steps, "ms_per_step": ms, "TFLOPs": tflops}))
        return 0

    # ---- end to end with cached preprocess (reference timing convention) ---
    cache = prepare_for_attention(qd, kd, vd, cfg)
    e2e_ms = _events_time(lambda: fake_quant_attention(qd, kd, vd, cfg, preprocess_cache=cache), 5, 2)
    full_ms = _events_time(lambda: fake_quant_attention(qd, kd, vd, cfg), 2, 1)
    del cache

    # ---- next to the path: the Wan call boundary and the diagnostics ---------
    from low_bit_fake_quant import wan_hook
    from low_bit_fake_quant.p_requant import p_requant_rows
    from low_bit_fake_quant.rowmax_counters import count_rowmax_updates
    extra = {}
    if n_real != s:
        wan_hook.set_quant_cfg(cfg)
        qv, kv, vv = qd[:, :n_real], kd[:, :n_real], vd[:, :n_real]
        extra["wan_hook_call_ms"] = _events_time(lambda: wan_hook.fake_or_sdpa_attention(qv, kv, vv), 2, 1)
        extra["wan_hook_note"] = f"unpadded N={n_real} through the hook (pad + uncached fake_quant_attention)"
        wan_hook.set_quant_cfg(None)
    if cfg.qk_quant == "fp8_block" and ops.rowmax is not None:
        cnt_ms = _events_time(lambda: count_rowmax_updates(ops, cfg, sm_scale=sm_scale, up_threshold=16.0,
                                                           down_threshold=32.0, use_estimate=True), 3, 1)
        c = count_rowmax_updates(ops, cfg, sm_scale=sm_scale, up_threshold=16.0, down_threshold=32.0,
                                 use_estimate=True)
        qk_flops = flops / 2
        extra["rowmax_count"] = {"ms": cnt_ms, "TFLOPs": qk_flops / (cnt_ms * 1e-3) / 1e12,
                                 "rule": "estimated up16 down32", "updates": c["updates"],
                                 "rescales": c["rescales"], "rows_with_update": c["rows_with_update"],
                                 "note": "QK-only pass; time includes the counter read-back"}
    from low_bit_fake_quant import blasst_skip
    hs = min(h, 8)
    qs, ks, vs = (t[:, :, :hs] for t in (qd, kd, vd))
    sim_s = _events_time(lambda: blasst_skip.simulate_workload(qs, ks, vs, skip_thresholds=[0.05],
                                                               levels=[blasst_skip.LEVEL_FP8_SKIP]), 1, 0) / 1e3
    sim = blasst_skip.simulate_workload(qs, ks, vs, skip_thresholds=[0.05], levels=[blasst_skip.LEVEL_FP8_SKIP])
    extra["blasst_tile_sim"] = {"heads": hs, "S": s, "threshold": 0.05, "seconds": sim_s,
                                "skip_rate": sim.skip_diagnostics[0.05].skip_rate,
                                "note": "skip rung of the tile-skip simulator: per-head quant, scan, keep, attend"}
    del qs, ks, vs, sim
    sc_probe = torch.randn(h, 256, 4096, device=dev)
    pr_ms = _events_time(lambda: p_requant_rows(sc_probe, sm_scale=sm_scale), 5, 2)
    extra["p_requant_rows"] = {"shape": list(sc_probe.shape), "ms": pr_ms,
                               "GBps": sc_probe.numel() * 5 / (pr_ms * 1e-3) / 1e9}
    del sc_probe

    # ---- prepass bandwidth: algorithmic bytes / time ------------------------
    elem = b * s * h * d
    # algorithmic minimum: every input read once, every output written once
    # (the qm.K_s kernel re-reads K to form K_s on the fly; that re-read is
    # traffic, not algorithmic bytes)
    quant_bytes = prepass_bytes(ops, 3 * elem * qd.element_size())
    prepass = {"quantise_qmk_ms": quant_ms, "quantise_qmk_GBps": quant_bytes / (quant_ms * 1e-3) / 1e9,
               "preprocess_ms": prep_ms, "algorithmic_bytes": quant_bytes,
               "note": "quantisers + qm.K_s table; algorithmic bytes (inputs read once, outputs written once) / time"}
    prepass["frac_of_hbm_peak"] = prepass["quantise_qmk_GBps"] / HBM_PEAK_GBS
    # the practical ceiling, measured in the same run: a 1 GiB device copy
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    copy_ms = _events_time(lambda: dst.copy_(src), 5, 2)
    del src, dst
    copy_gbs = 2 * (1 << 30) / (copy_ms * 1e-3) / 1e9
    prepass["copy_GBps"] = copy_gbs
    prepass["frac_of_copy_rate"] = prepass["quantise_qmk_GBps"] / copy_gbs
    # the ceiling from this library's own streaming kernels, same run
    stream = hbm_ceiling(dev)
    prepass["hbm_stream"] = stream
    prepass["frac_of_stream_copy"] = prepass["quantise_qmk_GBps"] / stream["copy"]["GBps"]
    # on the reference's own bytes: Q/K/V read, codes written, no correction table
    ref_bytes = 3 * elem * 2 + 3 * elem * 1
    prepass["reference_bytes"] = ref_bytes
    prepass["reference_bytes_GBps"] = ref_bytes / (quant_ms * 1e-3) / 1e9
    if cfg.q_kmeans_k is not None:
        # Q k-means alone (part of the uncached preprocess): `iters` assignment
        # passes (2 S K D flops per head each, fp32 VALU in a fixed order) and
        # iters - 1 centroid updates, each pass reading Q once
        from low_bit_fake_quant._ops import kmeans
        kk, it = cfg.q_kmeans_k, cfg.q_kmeans_iters
        km_ms = _events_time(lambda: kmeans(qd, kk, it, cfg.q_kmeans_seed), 3, 1)
        km_flops = it * 2.0 * s * kk * d * h * b
        km_bytes = (2 * it - 1) * elem * qd.element_size()
        prepass["kmeans"] = {"k": kk, "iters": it, "ms": km_ms,
                             "assign_TFLOPs": km_flops / (km_ms * 1e-3) / 1e12,
                             "frac_of_fp32_peak": km_flops / (km_ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS,
                             "GBps": km_bytes / (km_ms * 1e-3) / 1e9,
                             "note": "assignment flops (2 S K D per head and pass) against the fp32 peak; "
                                     "bytes = Q read once per pass"}
        log(f"k-means: {km_ms:.3f} ms ({prepass['kmeans']['assign_TFLOPs']:.1f} TFLOP/s assign, "
            f"{prepass['kmeans']['GBps']:.0f} GB/s)")

    cpu_baseline = None
    err = err_replay = None
    if not args.no_cpu and args.config in (1, 2, 3):
        log("cpu baseline / error sample ...")
        cpu_baseline, err, err_replay = cpu_baseline_and_error(q, k, v, cfg, out, n_real, args.cpu_rows,
                                                               sm_scale)
    others = None
    if not args.no_other_configs and args.heads == 0 and args.config == 2:
        del qd, kd, vd, ops, prep
        torch.cuda.empty_cache()
        others = other_configs([1, 3, 4], dev)
        others["path_a"] = path_a(dev)

    roof = {"bound": "mfma", "achieved": tflops, "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / FP8_PEAK_TFLOPS, "traffic": None,
            "kernel": "attn_fwd_kernel", "flops_per_launch": flops}
    roof["traffic"] = traffic_from_profile(args.config)
    line = {
        "metric": "attn TFLOPS & % FP8-MFMA peak at 40h x 32760 x d128; prepass HBM GB/s; err vs ref",
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (MFMA) / fp32 accumulate",
        "data": "synthetic (seeded CPU generator, Wan-shaped)",
        "config": {"workload": w.name, "B": b, "H": h, "N": n_real, "N_padded": s, "D": d,
                   "qk_quant": cfg.qk_quant, "fp8_block_size": cfg.fp8_block_size, "v_quant": cfg.v_quant,
                   "smoothing": cfg.smoothing, "q_kmeans_k": cfg.q_kmeans_k, "p_quant": cfg.p_quant,
                   "rowmax_mode": cfg.rowmax_mode, "blasst_lambda": cfg.blasst_lambda},
        "roofline": roof,
        "cpu_baseline": cpu_baseline,
        "prepass": prepass,
        "e2e_cached_ms": e2e_ms,
        "e2e_cached_TFLOPs": flops / (e2e_ms * 1e-3) / 1e12,
        "full_call_ms": full_ms,
        "err_vs_oracle": err,
        "err_vs_replay": err_replay,
        "other_configs": others,
        "next_to_path": extra,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
