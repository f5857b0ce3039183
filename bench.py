"""Decode-step benchmark of the EntmaxKV MI355X build.

Workload (the headline metric): B=8, H=32 (MHA), D=128, 32768-token prefill plus one
appended token, page size 16, fp16, alpha=1.5.  One step = one call of
``sparse_attention_decode_paged`` (token budget 1024, niter 2, the cache
already appended, as in the reference's tests/run_benchmarks.py), with every
input resident in HBM.  The Gaussian-aware step (tau_mode "corrected") on the
same shape is reported alongside, on keys drawn as in benchmark config 3
(per-head offsets, 2% outlier pages aligned with q; --gauss-keys iid for N(0, 1)).

value = effective bytes per step / step time, where the effective bytes are
the selected K and V rows, one criticality bound per (b, h, page, d), q and
out (the reference's accounting of the bytes a step must touch).

Prints one JSON line.  --gpus N > 1 is rejected: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--heads", type=int, default=32)
    p.add_argument("--kv-heads", type=int, default=None)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--kv-len", type=int, default=32768)
    p.add_argument("--budget", type=int, default=1024)
    p.add_argument("--niter", type=int, default=2)
    p.add_argument("--alpha", type=float, default=1.5)
    p.add_argument("--dtype", default="fp16", choices=["fp16", "bf16", "fp32"])
    p.add_argument("--no-graph", action="store_true", help="time eager launches only")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-gaussian", action="store_true")
    p.add_argument("--gauss-keys", choices=["c3", "iid"], default="c3",
                   help="keys of the Gaussian-aware step: c3 = N(mu_h, 1) per head with 2%% "
                        "outlier pages scaled x3 toward q (benchmark config 3), iid = N(0, 1)")
    p.add_argument("--only", choices=["topk", "gaussian", "criticality"], default=None,
                   help="run one step kind in a loop (for profilers)")
    p.add_argument("--config", choices=["headline", "c5", "dense", "rows"], default="headline",
                   help="c5: benchmark config 5 instead of the headline line (ragged batch, "
                        "B=32, 32 q / 8 kv heads, bf16, lengths ~ U[4096, 131072], 1%% outlier "
                        "pages x4, Gaussian alpha 1.5 with append over 16 consecutive steps); "
                        "dense: the dense (non-paged) decode over every token of the headline "
                        "shape; rows: row-wise entmax forward + backward")
    p.add_argument("--copy-calib-mib", type=int, default=0,
                   help="with --only: first copy a buffer of this many MiB (a copy kernel of "
                        "known traffic that scales rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def _time_loop(fn, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms


def _step_percentiles(fn, steps, stream):
    """Median and 90th percentile of single-step durations (us), each step
    bracketed by its own events (after the timed loops, not part of them)."""
    import torch
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for s, e in ev:
        s.record(stream)
        fn()
        e.record(stream)
    torch.cuda.synchronize()
    t = sorted(s.elapsed_time(e) * 1e3 for s, e in ev)
    return round(t[len(t) // 2], 2), round(t[(9 * len(t)) // 10], 2)


def _graphed(fn, stream):
    import torch
    g = torch.cuda.CUDAGraph()
    fn()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g.replay


def _gaussian_cache(B, H, Hkv, L, D, ps, dt, dev, q, kind):
    """Cache for the Gaussian-aware step (seeded, built on the device).

    c3: keys ~ N(mu_h, 1) with mu_h ~ N(0, 0.5) per (b, kv head); 2% of the
    pages of each (b, kv head), chosen at random, become 3 * (k + 4 q_hat),
    q_hat the unit query of the group's first head; values ~ N(0, 1).
    """
    import torch

    from entmaxkv_amd import PagedKVCache

    g = torch.Generator(device=dev)
    g.manual_seed(1)
    k = torch.randn(B, Hkv, L, D, device=dev, dtype=torch.float32, generator=g)
    if kind == "c3":
        k += torch.randn(B, Hkv, 1, 1, device=dev, generator=g) * math.sqrt(0.5)
        P = L // ps
        n_out = max(1, int(0.02 * P))
        G = H // Hkv
        qh = q[:, ::G, 0].float()
        qh = qh / qh.norm(dim=-1, keepdim=True)  # [B, Hkv, D]
        pages = torch.argsort(torch.rand(B, Hkv, P, device=dev, generator=g), dim=-1)[..., :n_out]
        kp = k[:, :, : P * ps].view(B, Hkv, P, ps, D)
        idx = pages[..., None, None].expand(B, Hkv, n_out, ps, D)
        sel = torch.gather(kp, 2, idx)
        sel = 3.0 * (sel + 4.0 * qh[:, :, None, None, :])
        kp.scatter_(2, idx, sel)
    k = k.to(dt)
    v = torch.randn(B, Hkv, L, D, device=dev, dtype=torch.float32, generator=g).to(dt)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(k, v)
    del k, v
    return cache


def _config5(a):
    """benchmark config 5: a ragged batch decoded with Gaussian-aware selection.

    B=32, H=32 query / 8 kv heads, D=128, bf16, page size 16; sequence
    lengths drawn from U[4096, 131072] (seeded, last pages partial); keys and
    values ~ N(0, 1) with 1% of each (b, kv head)'s pages scaled x4;
    alpha 1.5, tau_mode "corrected", append_cache=True.  One measurement is
    16 consecutive decode steps (each appends one token per sequence), after
    `warmup` untimed steps.  Bytes per step: k_mean + k_std of every
    statistics page, the selected K and V rows, the appended K/V rows, q and
    out.
    """
    import torch

    from entmaxkv_amd import PagedKVCache, sparse_attention_decode_gaussian_aware_entmax

    B, H, Hkv, D, ps, esz = 32, 32, 8, 128, 16, 2
    dt, dev = torch.bfloat16, torch.device("cuda:0")
    g = torch.Generator(device="cpu")
    g.manual_seed(5)
    lens = torch.randint(4096, 131072 + 1, (B,), generator=g)
    Lmax = int(lens.max())
    gd = torch.Generator(device=dev)
    gd.manual_seed(5)
    k = torch.randn(B, Hkv, Lmax, D, device=dev, dtype=dt, generator=gd)
    P = Lmax // ps
    n_out = max(1, P // 100)
    pages = torch.randint(0, P, (B, Hkv, n_out), device=dev, generator=gd)
    rows = (pages[..., None] * ps + torch.arange(ps, device=dev)).reshape(B, Hkv, -1)
    kp = torch.gather(k, 2, rows[..., None].expand(-1, -1, -1, D)) * 4.0
    k.scatter_(2, rows[..., None].expand(-1, -1, -1, D), kp)
    v = torch.randn(B, Hkv, Lmax, D, device=dev, dtype=dt, generator=gd)
    cache = PagedKVCache(page_size=ps, headroom=a.warmup + a.steps + 16)
    cache.initialize(k, v, seq_lens=lens)
    del k, v, kp
    torch.cuda.empty_cache()
    q = torch.randn(B, H, 1, D, device=dev, dtype=dt, generator=gd)
    kn = torch.randn(B, Hkv, 1, D, device=dev, dtype=dt, generator=gd)
    vn = torch.randn(B, Hkv, 1, D, device=dev, dtype=dt, generator=gd)
    out = torch.zeros_like(q)
    stream = torch.cuda.current_stream(dev)

    def step():
        sparse_attention_decode_gaussian_aware_entmax(q, cache, kn, vn, out, alpha=1.5,
                                                      tau_mode="corrected", append_cache=True)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_steps = 16
    sel_tok = 0.0
    stat_bytes = 0.0
    t0.record(stream)
    for _ in range(n_steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / n_steps
    # bytes of the last step (lengths grow by one per step: the same to 0.1%)
    lens_now = cache.seq_lens.long().cpu()
    Pb = (lens_now + ps - 1) // ps
    pfs = torch.where(Pb > 1, Pb - 1, Pb)
    lps = lens_now - (Pb - 1) * ps
    counts = cache.last_num_selected_per_head.long().cpu()
    sel_tok = float(((counts - 1).clamp(min=0) * ps + lps[:, None]).sum())
    stat_bytes = float(pfs.sum()) * Hkv * D * esz * 2
    step_bytes = stat_bytes + sel_tok * D * esz * 2 + 2 * B * H * D * esz + 2 * B * Hkv * D * esz
    gbs = step_bytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "decode-step us + effective KV GB/s (% HBM peak), benchmark config 5",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": n_steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 storage, f32 accumulate",
        "data": "synthetic N(0,1) q/k/v with 1% outlier pages x4, seed 5",
        "config": {"workload": "ragged Gaussian-aware decode, append each step", "batch": B,
                   "q_heads": H, "kv_heads": Hkv, "head_dim": D, "page_size": ps,
                   "seq_lens_min": int(lens_now.min()), "seq_lens_max": int(lens_now.max()),
                   "seq_lens_mean": round(float(lens_now.float().mean()), 1), "alpha": 1.5,
                   "tau_mode": "corrected", "timing": "eager, 16 consecutive steps",
                   "mean_selected_pages": round(float(counts.float().mean()), 2),
                   "bytes_per_step": step_bytes}}), flush=True)
    return 0


def _config_dense(a):
    """Dense (non-paged) decode at the headline shape: B=8, H=32, D=128, L=32768,
    fp16, alpha 1.5, niter 2, every token attended.  Algorithmic bytes per
    step: all K rows, the V rows of supported tokens (counted on the output's
    tau), q and out."""
    import torch

    from entmaxkv_amd.kernels import DenseDecodeWorkspace, sparse_attention_decode_orchestrator

    B, H, D, L, esz = a.batch, a.heads, a.head_dim, a.kv_len, 2
    dt, dev = torch.float16, torch.device("cuda:0")
    gd = torch.Generator(device=dev)
    gd.manual_seed(1)
    k = torch.randn(B, H, L, D, device=dev, dtype=dt, generator=gd)
    v = torch.randn(B, H, L, D, device=dev, dtype=dt, generator=gd)
    q = torch.randn(B, H, 1, D, device=dev, dtype=dt, generator=gd)
    out = torch.zeros_like(q)
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    taus = torch.empty(B, H, dtype=torch.float32, device=dev)
    ws = DenseDecodeWorkspace(B, H, L, dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        sparse_attention_decode_orchestrator(q, k, v, out, lens, None, alpha=a.alpha, niter=2,
                                             workspace=ws, taus_out=taus)

    ms = _time_loop(step, a.steps, a.warmup, stream)
    # supported tokens at the final tau (the V rows the decode reads)
    s = torch.einsum("bhd,bhld->bhl", q[:, :, 0].float(), k.float())
    s = s * ((a.alpha - 1.0) / math.sqrt(D))
    support = float((s > taus[..., None]).sum())
    step_bytes = B * H * L * D * esz + support * D * esz + 2 * B * H * D * esz
    gbs = step_bytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "dense decode-step us + effective KV GB/s (% HBM peak)",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16 storage, f32 accumulate",
        "data": "synthetic N(0,1) q/k/v, seed 1",
        "config": {"workload": "dense entmax decode (sparse_attention_decode_orchestrator)",
                   "batch": B, "heads": H, "head_dim": D, "kv_len": L, "alpha": a.alpha,
                   "niter": 2, "mean_support": round(support / (B * H), 1),
                   "bytes_per_step": step_bytes}}), flush=True)
    return 0


def _config_rows(a):
    """Row-wise entmax forward and backward over 16384 rows of 8192 fp16
    values (alpha 1.5).  Algorithmic bytes: forward reads x and writes y,
    backward reads y and dy and writes dx."""
    import torch

    from entmaxkv_amd.entmax import entmax_backward, entmax_forward

    R, N, esz = 16384, 8192, 2
    dev = torch.device("cuda:0")
    gd = torch.Generator(device=dev)
    gd.manual_seed(2)
    x = torch.randn(R, N, device=dev, dtype=torch.float16, generator=gd) * 3
    dy = torch.randn(R, N, device=dev, dtype=torch.float16, generator=gd)
    stream = torch.cuda.current_stream(dev)
    y = entmax_forward(x, 1.5)
    ms_f = _time_loop(lambda: entmax_forward(x, 1.5), a.steps, a.warmup, stream)
    ms_b = _time_loop(lambda: entmax_backward(y, dy, 1.5), a.steps, a.warmup, stream)
    fb, bb = 2.0 * R * N * esz, 3.0 * R * N * esz
    gf, gb = fb / (ms_f * 1e-3) / 1e9, bb / (ms_b * 1e-3) / 1e9
    print(json.dumps({
        "metric": "row-wise entmax forward / backward GB/s (% HBM peak)",
        "value": round(gf, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_f, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16 storage, f32 accumulate",
        "data": "synthetic N(0,9) x, N(0,1) dy, seed 2",
        "forward": {"us": round(ms_f * 1e3, 2), "GBs": round(gf, 1),
                    "pct_hbm_peak": round(100.0 * gf / HBM_PEAK_GBS, 2), "bytes": fb},
        "backward": {"us": round(ms_b * 1e3, 2), "GBs": round(gb, 1),
                     "pct_hbm_peak": round(100.0 * gb / HBM_PEAK_GBS, 2), "bytes": bb},
        "config": {"workload": "triton_entmax rows", "rows": R, "n": N, "alpha": 1.5}}),
        flush=True)
    return 0


def main():
    a = _args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not built)"}))
        return 2
    if a.config == "c5":
        return _config5(a)
    if a.config == "dense":
        return _config_dense(a)
    if a.config == "rows":
        return _config_rows(a)
    import numpy as np
    import torch

    from entmaxkv_amd import (PagedKVCache, sparse_attention_decode_gaussian_aware_entmax,
                              sparse_attention_decode_paged)

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[a.dtype]
    esz = torch.tensor([], dtype=dt).element_size()
    B, H, D, L, ps = a.batch, a.heads, a.head_dim, a.kv_len, 16
    Hkv = a.kv_heads or H
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    k = torch.randn(B, Hkv, L, D, device=dev, dtype=dt)
    v = torch.randn(B, Hkv, L, D, device=dev, dtype=dt)
    q = torch.randn(B, H, 1, D, device=dev, dtype=dt)
    k_new = torch.randn(B, Hkv, 1, D, device=dev, dtype=dt)
    v_new = torch.randn(B, Hkv, 1, D, device=dev, dtype=dt)
    cache = PagedKVCache(page_size=ps)
    cache.initialize(k, v)
    cache.append(k_new, v_new)
    del k, v
    torch.cuda.empty_cache()

    S = L + 1
    P = (S + ps - 1) // ps
    n_sel = min(a.budget // ps, P - 1)
    lps = S - (P - 1) * ps
    n_tok = n_sel * ps + lps
    cache_seqlens = torch.full((B,), n_tok, device=dev, dtype=torch.int32)
    q_seqlens = torch.full((B,), S, device=dev, dtype=torch.int32)
    out = torch.zeros_like(q)
    stream = torch.cuda.current_stream(dev)

    def topk_step():
        sparse_attention_decode_paged(q, cache, k_new, v_new, out, a.budget, cache_seqlens,
                                      q_seqlens, alpha=a.alpha, niter=a.niter, append_cache=False)

    def crit_only():
        cache.select_topk(q, n_sel)

    # effective (algorithmic) bytes: selected K+V rows, one bound per (b,h,page,d), q, out
    kv_bytes = B * Hkv * n_tok * D * esz * 2
    crit_bytes = B * H * (P - 1) * D * esz if Hkv == H else B * Hkv * (P - 1) * D * esz * 2
    io_bytes = 2 * B * H * D * esz
    step_bytes = kv_bytes + crit_bytes + io_bytes

    if a.only:
        if a.copy_calib_mib:
            n = a.copy_calib_mib * (1 << 20) // 4
            src = torch.ones(n, device=dev, dtype=torch.float32)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
        fn = {"topk": topk_step, "criticality": crit_only}.get(a.only)
        if a.only == "gaussian":
            gcache = _gaussian_cache(B, H, Hkv, S, D, ps, dt, dev, q, a.gauss_keys)

            def fn():
                sparse_attention_decode_gaussian_aware_entmax(q, gcache, k_new, v_new, out,
                                                              alpha=a.alpha, tau_mode="corrected")
        ms = _time_loop(fn, a.steps, a.warmup, stream)
        print(json.dumps({"only": a.only, "ms_per_step": ms}), flush=True)
        return 0

    ms_eager = _time_loop(topk_step, a.steps, a.warmup, stream)
    ms_graph = None
    if not a.no_graph:
        replay = _graphed(topk_step, stream)
        ms_graph = _time_loop(replay, a.steps, a.warmup, stream)
    # the same launch either way: report the faster timing (a replayed graph adds
    # a gap per replay when the step is a single kernel) and say which it is
    ms = ms_eager if ms_graph is None else min(ms_eager, ms_graph)
    timing = "hipGraph replay" if (ms_graph is not None and ms_graph <= ms_eager) else "eager"

    # Dominant (and only) kernel of the step: topk_decode_kernel (criticality,
    # top-k, tau and the weighted sum per workgroup).  Its average launch
    # duration is the step time of the replayed graph, timed with events on
    # the stream it is launched on.
    fused = B * Hkv >= 128
    roof_kernel = "topk_decode_kernel" if fused else "criticality_head_kernel + decode kernels"
    launch_gbs = step_bytes / (ms * 1e-3) / 1e9

    gauss = None
    if not a.no_gaussian:
        gcache = _gaussian_cache(B, H, Hkv, S, D, ps, dt, dev, q, a.gauss_keys)

        def gauss_step():
            sparse_attention_decode_gaussian_aware_entmax(q, gcache, k_new, v_new, out,
                                                          alpha=a.alpha, tau_mode="corrected")
        gms_eager = _time_loop(gauss_step, a.steps, a.warmup, stream)
        gms_graph = None
        if not a.no_graph:
            greplay = _graphed(gauss_step, stream)
            gms_graph = _time_loop(greplay, a.steps, a.warmup, stream)
        gP = gcache.num_pages
        glps = S - (gP - 1) * ps
        sel = gcache.last_num_selected_per_head.double()
        sel_tok = float(((sel - 1).clamp(min=0) * ps + glps).sum().item())
        # moments read once per kv head + the selected K rows (V only on the support,
        # counted in full as an upper bound of the algorithmic bytes)
        g_bytes = B * Hkv * (gP - 1) * D * esz * 2 + sel_tok * D * esz * 2 + io_bytes
        gms = gms_eager if gms_graph is None else min(gms_eager, gms_graph)
        gauss = {"keys": a.gauss_keys, "us_per_step": round(gms * 1e3, 2),
                 "us_eager": round(gms_eager * 1e3, 2),
                 "us_graph": None if gms_graph is None else round(gms_graph * 1e3, 2),
                 "effective_GBs": round(g_bytes / (gms * 1e-3) / 1e9, 1),
                 "pct_hbm_peak": round(100.0 * g_bytes / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                 "mean_selected_pages": round(float(sel.mean().item()), 2),
                 "bytes_per_step": g_bytes}

    cpu = None
    if not a.no_cpu_baseline:
        cpu = _cpu_baseline(a, esz, q, cache, step_bytes)

    value = step_bytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "decode-step us + effective KV GB/s (% HBM peak), B=8 H=32 D=128 L=32k alpha=1.5",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "us_per_step_eager": round(ms_eager * 1e3, 2),
        "us_per_step_graph": None if ms_graph is None else round(ms_graph * 1e3, 2),
        "us_step_median_p90": _step_percentiles(topk_step, min(a.steps, 200), stream),
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp16": "f16", "bf16": "bf16", "fp32": "f32"}[a.dtype] + " storage, f32 accumulate",
        "data": "synthetic N(0,1) q/k/v, torch.manual_seed(0)",
        "config": {"workload": "top-k paged sparse-entmax decode step", "batch": B, "q_heads": H,
                   "kv_heads": Hkv, "head_dim": D, "kv_len": S, "page_size": ps,
                   "token_budget": a.budget, "selected_tokens_per_head": n_tok,
                   "alpha": a.alpha, "niter": a.niter, "timing": timing,
                   "bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "kernel": roof_kernel,
                     "achieved": round(launch_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(launch_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "avg_launch_us": round(ms * 1e3, 2), "bytes_per_launch": step_bytes},
        "gaussian": gauss,
        "cpu_baseline": cpu,
        "build_id": _lib_build_id(),
    }
    headline = (B, H, Hkv, D, L, a.budget, a.dtype) == (8, 32, 32, 128, 32768, 1024, "fp16")
    traffic = _measured_traffic("topk_decode_kernel") if headline and fused else None
    if traffic:
        line["roofline"]["traffic"] = traffic
        line["roofline"]["frac_traffic"] = round(traffic / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    print(json.dumps(line), flush=True)
    return 0


def _lib_build_id():
    from entmaxkv_amd import _lib
    return _lib.build_id()


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "topk_decode_kernel_pmc_b8h32l32k.md")


def _measured_traffic(kernel_tag):
    """HBM bytes per launch of the roofline kernel at the headline shape.

    Read from the committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE,
    each scaled by the factor a copy kernel of known size gives).  None unless
    the summary names this kernel and the build id of the loaded library: a
    figure taken on another build of the kernels is not reported.
    """
    import re

    from entmaxkv_amd import _lib
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    k = re.search(r"^kernel:\s*(\S+)", text, re.M)
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    b = re.search(r"^build_id:\s*(\S+)", text, re.M)
    if not (k and m and b) or kernel_tag not in k.group(1) or b.group(1) != _lib.build_id():
        return None
    return int(m.group(1))


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads():
    """Host cores this process may use, at most 16 (the GPU box's CPU share
    for one GPU, whatever the machine's core count is)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _cpu_baseline(a, esz, q, cache, step_bytes):
    """The top-k step restated in PyTorch on the host (float32, every usable
    core), on the same cache contents as the GPU step: the full workload
    (all B), timed over a bounded sample of about 10 s.  The cache tensors are
    copied to host memory before the clock starts."""
    import torch

    from oracle import torch_cpu_step as T

    if (a.kv_heads or a.heads) != a.heads:
        return None  # the restatement is MHA only
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    qc = q[:, :, 0].float().cpu()
    kc, vc = cache.k_cache.cpu(), cache.v_cache.cpu()
    kmin, kmax = cache.k_min.cpu(), cache.k_max.cpu()
    T.topk_decode_step(qc, kc, vc, kmin, kmax, a.budget, 16, a.alpha)  # warm-up
    reps = 0
    t1 = time.perf_counter()
    while True:
        T.topk_decode_step(qc, kc, vc, kmin, kmax, a.budget, 16, a.alpha)
        reps += 1
        if time.perf_counter() - t1 >= 10.0:
            break
    sec = (time.perf_counter() - t1) / reps
    return {"value": round(step_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"the full workload (B={a.batch}, H={a.heads}, L={a.kv_len + 1}), PyTorch "
                      f"float32 restatement of the step (oracle/torch_cpu_step.py) with "
                      f"torch.set_num_threads({threads}) on {_cpu_model()}; {reps} steps in "
                      f"~10 s, {sec * 1e3:.1f} ms per step",
            "us_per_step": round(sec * 1e6, 1), "cpu_model": _cpu_model()}


if __name__ == "__main__":
    raise SystemExit(main())
