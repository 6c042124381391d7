#!/usr/bin/env python
"""Benchmark of the fused warm-tier dequant + decode attention on one MI355X.

One step = one decode step of one attention layer for every sequence of the
workload (one new query token per sequence) over its hot + warm window, run
by the fused HIP kernel with the quantized KV cache already resident in HBM.

Prints ONE JSON line:
  value        decode tokens/s (batch / wall-clock seconds per step)
  roofline     algorithmic HBM bytes per launch / HIP-event kernel time,
               against MI355X's 8 TB/s
  cpu_baseline the torch-CPU restatement of the reference path on this
               host's cores over a bounded sample of sequences
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # the GPU raises its clocks over the first tens of milliseconds of work;
    # whatever --warmup asks for, warm-up also runs until WARMUP_FLOOR_MS of
    # launches have completed (warm_up below), so that the timed region
    # starts at the steady state
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--workload", default="batched_32x32k")
    ap.add_argument("--splits", type=int, default=0, help="token splits per (sequence, KV head); 0 = auto")
    ap.add_argument("--cpu-sample", type=int, default=4, help="sequences timed on the CPU baseline")
    ap.add_argument("--cpu-repeats", type=int, default=32)
    ap.add_argument("--stream-steps", type=int, default=600,
                    help="long-context workload: streaming appends timed after the decode line (0 = skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="batched_32x32k: skip the encode_4k and longctx_128k sub-records timed after it")
    ap.add_argument("--cpu-budget", type=float, default=1.0,
                    help="scale of the CPU baselines' time budgets")
    ap.add_argument("--no-exact", action="store_true", help="skip timing the exact codebook K path beside the tables")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    return ap.parse_args(argv)


# Measured on MI355X (one launch of the batch 32 x 32K decode step takes
# 0.167 ms once the clocks are up): after 5 warm-up launches the next 40 took
# 0.21 ms each, after 400 (about 70 ms) 0.167 ms.  The floor is well past that.
WARMUP_FLOOR_MS = 300.0


def warm_up(fn, steps: int, floor_ms: float = WARMUP_FLOOR_MS, batch: int = 64) -> dict:
    """Run ``fn`` ``steps`` times, then more (in batches, synchronized) until
    at least ``floor_ms`` of wall-clock time has passed since the first call.
    Returns the steps actually run and the time they took."""
    import torch

    t0 = time.perf_counter()
    n = 0
    for _ in range(steps):
        fn()
        n += 1
    torch.cuda.synchronize()
    while (time.perf_counter() - t0) * 1e3 < floor_ms:
        for _ in range(batch):
            fn()
        n += batch
        torch.cuda.synchronize()
    return {"steps_run": n, "ms": round((time.perf_counter() - t0) * 1e3, 1), "floor_ms": floor_ms}


def copy_calibration(mib: int, reps: int = 5) -> dict:
    """A device-to-device copy of exactly ``mib`` MiB, ``reps`` times: its
    per-dispatch FETCH_SIZE and WRITE_SIZE should each read ``mib * 1024`` KiB."""
    import torch

    n = mib << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    ok = bool(torch.equal(src, dst))
    return {"copy_calibration_bytes": n, "expected_kib_per_dispatch": n / 1024, "reps": reps, "ok": ok}


def fit_quantizer(cfg, x, g, w, dev):
    """k-means PQ codebooks on a seeded subsample, then RVQ codebooks on its PQ residual."""
    import torch
    from apple_amd import kernels as K
    from apple_amd.calibrate import fit_codebooks
    from apple_amd.quantization import HybridQuantizerMLX

    flat = x.reshape(-1, x.shape[-1])
    n = flat.shape[0]
    if n > w.kmeans_sample:
        idx = torch.randperm(n, generator=g)[: w.kmeans_sample].to(dev)
        flat = flat[idx]
    flat = flat.contiguous()
    pq_cb, _ = fit_codebooks(flat, w.pq_subspaces, w.pq_centroids, w.kmeans_iters, g)
    rvq_cb = None
    if w.rvq_subspaces:
        _, r1 = K.pq_encode(flat, pq_cb)
        rvq_cb, _ = fit_codebooks(r1, w.rvq_subspaces, w.rvq_centroids, w.kmeans_iters, g)
    return HybridQuantizerMLX(cfg, device=dev, pq_codebooks=pq_cb, rvq_codebooks=rvq_cb)


def setup_decode(w, dev):
    import torch
    from apple_amd.batched import RFSNBatchedKVCache
    from apple_amd.workloads import make_sequence

    cfg = w.config()
    cache = RFSNBatchedKVCache(cfg, w.batch, device=dev)
    qs = []
    t0 = time.time()
    for b in range(w.batch):
        k, v, q, g = make_sequence(w, b)
        kd, vd = k.to(dev), v.to(dev)
        kq = fit_quantizer(cfg, kd[: w.warm], g, w, dev)
        vq = fit_quantizer(cfg, vd[: w.warm], g, w, dev)
        cache.prefill(b, kd, vd, kq, vq)
        qs.append(q)
        del kd, vd
        if b == 0 or (b + 1) % 8 == 0:
            log(f"sequence {b + 1}/{w.batch} encoded ({time.time() - t0:.1f} s)")
    torch.cuda.synchronize()
    return cache, torch.stack(qs).to(dev)


def exact_path(w, cache, q, gpu_out, steps: int, dev) -> dict:
    """The exact codebook K path timed beside the score tables: the same
    sequences and codebooks prefilled into a cache that rebuilds K^ from the
    codebooks (``fused_score_tables=False``), its kernel time over ``steps``
    launches (HIP events on the launch stream), and its largest output
    difference from the tables' output."""
    import dataclasses

    import torch
    from apple_amd.batched import RFSNBatchedKVCache
    from apple_amd.workloads import make_sequence

    cfg = dataclasses.replace(cache.config, fused_score_tables=False)
    exact = RFSNBatchedKVCache(cfg, w.batch, device=dev)
    for b in range(w.batch):
        k, v, _, _ = make_sequence(w, b)
        exact.prefill(b, k.to(dev), v.to(dev), *cache.quantizers[b])
    out = torch.empty_like(q)
    launch = exact.prepare(q, out=out)
    warm_up(launch, 10)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        launch()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    achieved = w.bytes_per_step() / (ms * 1e-3) / 1e9
    return {"k_scoring": "codebook K^ rows (exact)", "kernel_ms": round(ms, 5),
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "max_abs_vs_tables": float((out.float() - gpu_out.float()).abs().max())}


def cpu_baseline(w, cache, q, gpu_out, sample, repeats, threads=None):
    """Time the torch-CPU restatement of the path on a bounded sample, on
    every host core (or ``threads``)."""
    import torch
    from oracle import cpu_baseline as cb

    cores = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    total, n, max_err = 0.0, 0, 0.0
    for b in range(min(sample, w.batch)):
        nw, nh = cache.num_warm[b], cache.num_hot[b]
        codes = {kv: {k: t.cpu() for k, t in cache.plain_codes(kv, b).items() if t is not None}
                 for kv in ("k", "v")}
        cbs = {k: v[b].cpu() for k, v in cache.cb.items()}
        hk, hv = cache.hot_k[b, :, :nh].cpu(), cache.hot_v[b, :, :nh].cpu()
        qb = q[b:b + 1].cpu()
        out = cb.decode_step(qb, hk, hv, codes["k"], codes["v"], cbs, w.head_dim ** -0.5, w.block)  # warm-up
        t0 = time.perf_counter()
        for _ in range(repeats):
            out = cb.decode_step(qb, hk, hv, codes["k"], codes["v"], cbs, w.head_dim ** -0.5, w.block)
        total += time.perf_counter() - t0
        n += repeats
        max_err = max(max_err, float((out.float() - gpu_out[b:b + 1].float().cpu()).abs().max()))
    per_token = total / n
    return {"value": 1.0 / per_token, "unit": "decode tokens/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{min(sample, w.batch)} of {w.batch} sequences x {repeats} repeats, one decode step each "
                      f"(full {w.context}-token window, torch-CPU F.embedding decode + fp32 blockwise "
                      f"attention, block {w.block})",
            "seconds": round(total, 2)}, max_err


MFMA_PEAK_TFLOPS = 2500.0  # dense fp16


def bench_encode(w, args, dev) -> dict:
    """Warm-tier compression throughput: one step encodes one chunk of
    ``w.context`` tokens x ``w.kv_heads`` heads for K and for V (PQ, then the
    subspace RVQ stage on the PQ residual, then the top-k sparse residual)."""
    import torch
    from apple_amd import kernels as K
    from apple_amd.workloads import make_sequence

    cfg = w.config()
    k, v, _, g = make_sequence(w, 0)
    kd, vd = k.to(dev), v.to(dev)
    kq = fit_quantizer(cfg, kd, g, w, dev)
    vq = fit_quantizer(cfg, vd, g, w, dev)
    fmt = kq.warm_format()
    xs = [(t.reshape(-1, w.head_dim).contiguous(), qz) for t, qz in ((kd, kq), (vd, vq))]
    cbs = [(qz.pq.codebooks, qz.rvq.codebooks if fmt.rvq_subspaces else None) for _, qz in xs]

    jobs = [(x, pcb, rcb) for (x, _), (pcb, rcb) in zip(xs, cbs)]

    def step():  # K and V of the chunk in one launch
        K.warm_encode_batch(jobs, fmt)

    warm = warm_up(step, args.warmup)
    steps = max(args.steps, 256)  # one chunk is microseconds: time at least 256 back to back
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"timing {steps} encode steps")
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    kernel_ms = start.elapsed_time(end) / steps
    pct = step_percentiles(step, steps)
    vectors = 2 * w.context * w.kv_heads
    # algorithmic contraction flops: 2 * C * D per vector and stage
    flops = vectors * 2 * w.head_dim * (w.pq_centroids + (w.rvq_centroids if w.rvq_subspaces else 0))
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    result = {
        "metric": "warm-tier encode vectors/s (PQ+RVQ+top-k, MFMA nearest-centroid search), 1 GPU",
        "value": round(vectors / (kernel_ms * 1e-3), 1),
        "unit": "vectors/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_run": warm,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) K/V with per-channel scale U(0.5,2); k-means codebooks)",
        "config": {"workload": w.name, "chunk_tokens": w.context, "kv_heads": w.kv_heads, "head_dim": w.head_dim,
                   "vectors_per_step": vectors,
                   "format": f"PQ M{w.pq_subspaces}x{w.pq_centroids}"
                             + (f" + RVQ M{w.rvq_subspaces}x{w.rvq_centroids}" if w.rvq_subspaces else "")
                             + (f" + top-{w.sparse_k} sparse" if w.sparse_k else "")},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_PEAK_TFLOPS, 5), "traffic": None, "kernel_ms": round(kernel_ms, 5),
                     "kernel_ms_percentiles": pct,
                     "flops_per_step": flops},
    }
    if not args.no_cpu:
        log("CPU baseline")
        result["cpu_baseline"] = encode_cpu_baseline(w, xs, cbs, fmt.sparse_k, budget_s=10.0 * args.cpu_budget)
        four = encode_cpu_baseline(w, xs, cbs, fmt.sparse_k, threads=4, budget_s=4.0 * args.cpu_budget)
        result["cpu_baseline"]["at_4_threads"] = {k: four[k] for k in ("value", "cores", "seconds")}
    return result


def bench_ref(w, args, dev) -> dict:
    """Decode step over reference-format tiers: one query per head attends
    ``w.hot`` exact tokens and ``w.warm`` PQ + gated-RVQ tokens, decoded in
    registers by rfsn_ref_attention.  Beside it: the decode-then-attend path
    it replaces (decode_ref of the warm K and V into HBM, concatenation,
    blockwise attention)."""
    import dataclasses

    import numpy as np
    import torch
    from apple_amd import kernels as K
    from apple_amd.storage import CompressedTensorMLX, RFSNConfig

    H, D, M, C, L, Cr = w.heads, w.head_dim, w.pq_subspaces, w.pq_centroids, w.rvq_layers, w.rvq_centroids
    d = D // M
    g = torch.Generator("cpu").manual_seed(17)
    randn16 = lambda *shape, s=1.0: (torch.randn(*shape, generator=g) * s).half()
    pq_cb = randn16(M, C, d, s=(2.0 / d) ** 0.5)
    rvq_cb = randn16(L, Cr, D, s=(2.0 / D) ** 0.5)
    rvq_cb[:, 0] = 0
    hot_k, hot_v = randn16(H, w.hot, D), randn16(H, w.hot, D)  # the cache's hot ring [H][cap][D]
    q = randn16(1, H, D)
    rng = np.random.default_rng(17)
    n = w.warm * H
    stores = []
    for _ in range(2):
        pq = torch.from_numpy(rng.integers(0, C, (w.warm, H, M), dtype=np.uint8))
        rvq = torch.from_numpy(rng.integers(0, Cr, (n, L), dtype=np.uint16))
        offs = torch.arange(n, dtype=torch.int32)
        stores.append((pq, rvq, offs))
    dv = lambda t: t.to(dev)
    dstores = [CompressedTensorMLX(pq_codes=dv(pq), rvq_codes=dv(rvq), rvq_mask=torch.ones((w.warm, H), dtype=torch.bool,
                                                                                             device=dev),
                                   rvq_offsets=dv(offs), num_heads=H) for pq, rvq, offs in stores]
    hk, hv, qd = dv(hot_k), dv(hot_v), dv(q)
    cbd, rcbd = dv(pq_cb), dv(rvq_cb)
    hot = K.ref_exact_segment(hk, hv, hk.stride(1), hk.stride(0), 0, w.hot, 0)
    segs = [hot, K.ref_store_segment(dstores[0], dstores[1], 0, w.warm, w.hot)]
    # the cache's decode step reads its warm codes from a head-major copy of
    # the stores, made once per store version (outside the step; the copy's
    # own time is the best of 3 rebuilds after a first, warm-up one)
    segs_hm = [hot, K.ref_store_segment(dstores[0], dstores[1], 0, w.warm, w.hot, head_major=True)]
    head_major_ms = float("inf")
    for _ in range(3):
        torch.cuda.synchronize()
        t_hm = time.perf_counter()
        K.copy_head_major(dstores[0])
        K.copy_head_major(dstores[1])
        torch.cuda.synchronize()
        head_major_ms = min(head_major_ms, (time.perf_counter() - t_hm) * 1e3)
    out = torch.empty_like(qd)
    scale = D ** -0.5
    # the decode step as the cache issues it: score tables for the coded
    # tokens under the drift guard at the config's default tolerance (a group
    # whose estimate exceeds it decodes them instead); the exact decode of
    # every coded vector beside it
    tol = next(f.default for f in dataclasses.fields(RFSNConfig) if f.name == "score_table_tolerance")
    stats = K.ref_table_stats(cbd, cbd, rcbd, rcbd)
    drift = torch.empty((1, H), dtype=torch.float32, device=dev)
    common = dict(kv_heads=H, scale=scale, causal=False, qpos=None, k_pq_cb=cbd, v_pq_cb=cbd,
                  k_rvq_cb=rcbd, v_rvq_cb=rcbd)
    fused = K.ref_prepare(qd, out=out, segments=segs_hm, score_tables=tol, table_stats=stats, drift=drift, **common)
    xout = torch.empty_like(qd)
    exact = K.ref_prepare(qd, out=xout, segments=segs, **common)

    def materialized():
        dk = K.decode_ref(dstores[0].pq_codes.reshape(n, M), cbd, dstores[0].rvq_codes, dstores[0].rvq_offsets, rcbd)
        dvv = K.decode_ref(dstores[1].pq_codes.reshape(n, M), cbd, dstores[1].rvq_codes, dstores[1].rvq_offsets,
                           rcbd)
        keys = torch.cat([hk.permute(1, 0, 2), dk.view(w.warm, H, D)], 0)
        values = torch.cat([hv.permute(1, 0, 2), dvv.view(w.warm, H, D)], 0)
        return K.blockwise_attention(qd, keys, values, scale, False, None)

    log(f"workload {w.name}: H={H} D={D} hot={w.hot} warm={w.warm} PQ {M}x{C} RVQ {L}x{Cr}")
    warm = warm_up(fused, args.warmup)
    steps = args.steps
    stream = torch.cuda.current_stream()
    ms_per_step, kernel_ms = _timed(fused, steps, stream)
    pct = step_percentiles(fused, min(steps, 100))
    warm_up(exact, 20)
    x_ms, x_kernel_ms = _timed(exact, steps, stream)
    mat_out = materialized()
    warm_up(materialized, 20, floor_ms=50.0, batch=4)
    mat_ms, mat_kernel_ms = _timed(materialized, max(steps // 4, 10), stream)
    err = float((out.float() - mat_out.float()).abs().max())
    x_err = float((xout.float() - mat_out.float()).abs().max())
    algo = w.bytes_per_step()
    gbs = algo / (kernel_ms * 1e-3) / 1e9
    result = {
        "metric": "decode attn tokens/s + HBM GB/s (reference-format PQ+gated-RVQ dequant-attn), 1 GPU",
        "value": round(w.context / (kernel_ms * 1e-3), 1),
        "unit": "decode tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_run": warm,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) hot K/V and query; uniform random PQ/RVQ codes, every row active)",
        "config": {"workload": w.name, "heads": H, "head_dim": D, "context": w.context, "hot": w.hot,
                   "warm": w.warm, "format": f"PQ M{M}x{C} + gated RVQ {L}x{Cr} (reference format)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 5),
                     "traffic": traffic_from_profiles(w.name, "ref_attn_{}_kernel_trace.md", "traffic_bytes_per_step"),
                     "kernel_ms": round(kernel_ms, 5),
                     "kernel_ms_percentiles": pct, "bytes_per_step": algo,
                     "rvq_codeword_bytes_per_step": 2 * w.warm * H * L * D * 2},
        "materialized_path": {"kernel_ms": round(mat_kernel_ms, 5), "ms_per_step": round(mat_ms, 5),
                              "speedup": round(mat_kernel_ms / kernel_ms, 2), "max_abs_vs_fused": err},
        "score_tables": {"used": fused.score_tables, "tolerance": tol,
                         "max_estimate": float(drift.max()) if fused.score_tables else None,
                         "heads_decoded_exactly": int((drift > tol).sum()) if fused.score_tables else None,
                         "code_rows": "head-major copy of the warm stores",
                         "head_major_copy_ms": round(head_major_ms, 4)},
        "exact_decode_path": {"kernel_ms": round(x_kernel_ms, 5), "ms_per_step": round(x_ms, 5),
                              "speedup_of_tables": round(x_kernel_ms / kernel_ms, 2),
                              "max_abs_vs_materialized": x_err},
    }
    if not args.no_cpu:
        from oracle import cpu_baseline as cb

        log("CPU baseline")
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        hs = 4  # a sample of heads: the step's cost is linear in heads
        hk_c, hv_c = hot_k[:hs].permute(1, 0, 2).contiguous(), hot_v[:hs].permute(1, 0, 2).contiguous()
        warm_c = []
        for pq, rvq, offs in stores:
            keep = torch.arange(w.warm * H).reshape(w.warm, H)[:, :hs].reshape(-1)
            warm_c.append({"pq": pq[:, :hs].contiguous(), "rvq": rvq[keep].contiguous(),
                           "offsets": torch.arange(w.warm * hs, dtype=torch.int32)})
        cbs = {"pq": pq_cb, "rvq": rvq_cb}
        ref = cb.ref_decode_step(q[:, :hs], hk_c, hv_c, warm_c[0], warm_c[1], cbs, scale, 128)
        cpu_err = float((out[:, :hs].float().cpu() - ref.float()).abs().max())
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0 * args.cpu_budget or reps == 0:
            cb.ref_decode_step(q[:, :hs], hk_c, hv_c, warm_c[0], warm_c[1], cbs, scale, 128)
            reps += 1
        sec = (time.perf_counter() - t0) / reps * (H / hs)
        result["cpu_baseline"] = {"value": round(w.context / sec, 2), "unit": "decode tokens/s", "cores": cores,
                                  "kind": "port", "cpu_model": cpu_model(),
                                  "sample": f"{hs} of {H} heads, {reps} steps, scaled to {H} heads: torch-CPU "
                                            f"F.embedding PQ + gated RVQ decode, then blockwise attention "
                                            f"(block 128); max-abs vs the GPU {cpu_err:.2e}"}
    return result


def bench_refencode(w, args, dev) -> dict:
    """Warm-tier encode in the reference's own format at its default
    configuration: one chunk of ``w.context`` tokens x ``w.heads`` heads
    through HybridQuantizerMLX.encode (quantization.py:305-308): PQ, the norm
    gate and its compaction (one host sync for the active count, as the
    reference's np.asarray(mask)), then the full-dimension RVQ stages.  The
    roofline is the RVQ search kernel's (the dominant one): its algorithmic
    flops 2 * C * D per active row and stage over its own HIP-event time."""
    import torch
    from apple_amd import _lib as L
    from apple_amd import kernels as K
    from apple_amd.quantization import HybridQuantizerMLX
    from apple_amd.storage import RFSNConfig

    H, D, M, C, Ls, Cr = w.heads, w.head_dim, w.pq_subspaces, w.pq_centroids, w.rvq_layers, w.rvq_centroids
    cfg = RFSNConfig(hidden_dim=H * D, num_heads=H, head_dim=D, num_subspaces=M, subspace_dim=D // M,
                     pq_bits=(C - 1).bit_length(), num_rvq_layers=Ls, rvq_codebook_size=Cr)
    g = torch.Generator("cpu").manual_seed(17)
    qz = HybridQuantizerMLX(cfg, device=dev, generator=g)  # codebooks drawn as at quantization.py:110-115, 190-197
    scale = torch.rand((H, D), generator=g) * 1.5 + 0.5
    x = (torch.randn((w.context, H, D), generator=g) * scale).half().reshape(-1, D)
    xd = x.to(dev)
    n = x.shape[0]

    def step():
        return qz.encode(xd)

    log(f"workload {w.name}: {n} vectors, head_dim {D}, PQ {M}x{C}, RVQ {Ls}x{Cr}, threshold "
        f"{cfg.rvq_sparsity_threshold}")
    warm = warm_up(step, args.warmup)
    steps = max(args.steps // 10, 10)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        pq, rvq, mask, offs = step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    a = int(offs.numel())
    # the RVQ search kernel alone, on its stream, over the step's active rows
    _, resid = K.pq_encode(xd, qz.pq.codebooks)
    lib = L.load()
    wsb = lib.rfsn_rvq_encode_full_workspace_bytes(a, D, Ls, Cr)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    codes = torch.empty((a, Ls), dtype=torch.uint16, device=dev)
    cb = qz.rvq.codebooks.contiguous()
    stream = torch.cuda.current_stream()

    def rvq_only():
        L.call("rfsn_rvq_encode_full", resid.data_ptr(), D, D, offs.data_ptr(), a, cb.data_ptr(), Ls, Cr,
               codes.data_ptr(), ws.data_ptr() if wsb else None, wsb, stream.cuda_stream)

    rvq_only()
    torch.cuda.synchronize()
    same = bool(torch.equal(codes, rvq))
    _, rvq_ms = _timed(rvq_only, steps, stream)
    pct = step_percentiles(rvq_only, steps)
    flops = a * Ls * Cr * D * 2
    tflops = flops / (rvq_ms * 1e-3) / 1e12
    result = {
        "metric": "reference-format encode vectors/s (PQ + gated full-dimension RVQ, MFMA search), 1 GPU",
        "value": round(n / (ms_per_step * 1e-3), 1),
        "unit": "vectors/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_run": warm,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) K with per-channel scale U(0.5,2); codebooks drawn as the reference "
                "initialises them)",
        "config": {"workload": w.name, "vectors_per_step": n, "heads": H, "head_dim": D,
                   "format": f"PQ M{M}x{C} + gated RVQ {Ls}x{Cr}, threshold {cfg.rvq_sparsity_threshold}",
                   "active_rows": a},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_PEAK_TFLOPS, 5), "traffic": None, "kernel": "rvq_mfma_kernel<128>",
                     "kernel_ms": round(rvq_ms, 5), "kernel_ms_percentiles": pct, "flops_per_launch": flops,
                     "rows_per_s": round(a / (rvq_ms * 1e-3), 1), "codes_match_step": same},
    }
    if not args.no_cpu:
        from oracle import cpu_baseline as cbl

        log("CPU baseline")
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        sample = 2048
        xs, pcb, rcb = x[:sample], qz.pq.codebooks.cpu(), qz.rvq.codebooks.cpu()
        _, ccodes, _, _ = cbl.ref_encode(xs, pcb, rcb, cfg.rvq_sparsity_threshold)
        agree = float((ccodes == rvq[:ccodes.shape[0]].cpu().long()).float().mean()) if a >= sample else None
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0 * args.cpu_budget or reps == 0:
            cbl.ref_encode(xs, pcb, rcb, cfg.rvq_sparsity_threshold)
            reps += 1
        sec = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(sample * reps / sec, 1), "unit": "vectors/s", "cores": cores,
                                  "kind": "port", "cpu_model": cpu_model(),
                                  "sample": f"the chunk's first {sample} vectors, {reps} times: torch-CPU cdist^2 "
                                            f"PQ, norm gate, {Ls} chunked (|x|^2 - 2xc) + |c|^2 stages",
                                  "seconds": round(sec, 2), "codes_agree_with_gpu": agree}
    return result


def encode_cpu_baseline(w, xs, cbs, k: int, threads=None, budget_s: float = 10.0) -> dict:
    """The step's K and V chunks encoded by the torch-CPU restatement of the
    reference's PyTorch encode (fp32 cdist^2 + argmin per subspace, both
    stages, then top-k), repeated until ``budget_s`` seconds have passed, on
    every host core (or ``threads``)."""
    import torch
    from oracle import cpu_baseline as cb

    cores = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    host = [(x.cpu(), pcb.cpu(), None if rcb is None else rcb.cpu()) for (x, _), (pcb, rcb) in zip(xs, cbs)]
    for x, pcb, rcb in host:  # warm-up
        cb.warm_encode(x[:1024], pcb, rcb, k)
    n, t0 = 0, time.perf_counter()
    while True:
        for x, pcb, rcb in host:
            cb.warm_encode(x, pcb, rcb, k)
            n += x.shape[0]
        sec = time.perf_counter() - t0
        if sec >= budget_s:
            break
    return {"value": round(n / sec, 1), "unit": "vectors/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"the step's {2 * w.context * w.kv_heads} K and V vectors, {n // (2 * w.context * w.kv_heads)} "
                      f"times: torch-CPU fp32 cdist^2 + argmin per subspace (PQ, then RVQ on the residual), "
                      f"then top-{k} |r2|",
            "seconds": round(sec, 2)}


def step_percentiles(fn, steps):
    """p10 / p50 / p90 of per-call times (ms), from one event between each
    pair of back-to-back calls on the launch stream (a pass of its own)."""
    import torch

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(steps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    d = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    pick = lambda f: round(d[min(len(d) - 1, int(f * len(d)))], 5)
    return {"p10": pick(0.1), "p50": pick(0.5), "p90": pick(0.9)}


def device_copy_gbs(mib: int = 1024, reps: int = 10) -> float:
    """Measured device-to-device copy bandwidth, read + write bytes per second (GB/s)."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize()
    gbs = 2 * n * reps / (s.elapsed_time(e) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return round(gbs, 1)


def device_read_gbs(gib: int = 4, blocks: int = 65536, reps: int = 10) -> float:
    """Measured read-only HBM stream (rfsn_read_stream over ``gib`` GiB), GB/s:
    the ceiling a read-dominated kernel can reach on this device."""
    import torch
    from apple_amd import _lib as L

    n = gib << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    out = torch.empty(blocks, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        L.call("rfsn_read_stream", src.data_ptr(), n, out.data_ptr(), blocks, s)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        L.call("rfsn_read_stream", src.data_ptr(), n, out.data_ptr(), blocks, s)
    e1.record()
    torch.cuda.synchronize()
    gbs = n * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, out
    torch.cuda.empty_cache()
    return round(gbs, 1)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, steps, stream=None):
    """(host ms per call, HIP-event ms per call on ``stream``) over ``steps`` back-to-back calls."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps, start.elapsed_time(end) / steps


def bench_longctx(w, args, dev) -> dict:
    """Long-context decode with a cold tier: one sequence of ``w.context``
    tokens; the newest ``w.hot`` exact and the next ``w.warm`` encoded in HBM,
    the older tokens encoded in pinned host memory in ``w.cold_chunk``-token
    chunks.  The window is hot + warm + the ``w.cold_attended`` chunks the
    router ranks nearest the query.  ``value`` is the step with those chunks
    resident in device slots (a decode loop's steady state); the step that
    copies all of them in (side-stream copies overlapped with the attention
    over the resident part) is reported beside it."""
    import torch
    from apple_amd.cache import RFSNv10KVCacheMLX
    from apple_amd.storage import AsyncHierarchicalRouterMLX
    from apple_amd.workloads import make_sequence

    cfg = w.config()
    k, v, q, g = make_sequence(w, 0)
    kd, vd = k.to(dev), v.to(dev)
    kq = fit_quantizer(cfg, kd[w.cold:w.cold + w.warm], g, w, dev)
    vq = fit_quantizer(cfg, vd[w.cold:w.cold + w.warm], g, w, dev)
    cache = RFSNv10KVCacheMLX(cfg, device=dev, cold_slots=max(32, w.cold_attended))
    t0 = time.time()
    cache.update(kd, vd, (kq, vq))
    torch.cuda.synchronize()
    log(f"cache filled: hot {cache.num_hot}, warm {cache.num_warm}, cold {cache.num_cold} in "
        f"{len(cache.cold_chunk_metadata)} pinned chunks ({time.time() - t0:.1f} s)")
    del kd, vd
    router = AsyncHierarchicalRouterMLX(cfg).bind(cache)
    ids = router.rank(w.context - 1, w.context)[:w.cold_attended]
    qd = q[None].to(dev).contiguous()

    # steady state: the router's chunks resident in device slots, one launch per step
    cache.prefetch_cold_chunks(ids)
    out = torch.empty_like(qd)
    launch = cache.prepare(qd, causal=True, cold_chunks=ids, splits=args.splits, out=out)
    warm = warm_up(launch, args.warmup)
    log(f"timing {args.steps} steps (cold chunks resident)")
    ms_per_step, kernel_ms = _timed(launch, args.steps)
    pct = step_percentiles(launch, args.steps)

    # every step copies the chunks in: resident part || copies, then the copied chunks + merge
    cache.evict_cold_slots()
    out2 = torch.empty_like(qd)
    step = cache.prepare(qd, causal=True, cold_chunks=ids, out=out2)
    for _ in range(args.warmup):
        step()
    log(f"timing {args.steps} steps (cold chunks copied in every step)")
    refetch_host_ms, refetch_ms = _timed(step, args.steps)
    side = torch.cuda.ExternalStream(step.side.stream)

    def copies_only():
        step.issue_copies()

    copy_host_ms, copy_ms = _timed(copies_only, args.steps, side)
    _, resident_ms = _timed(step.launches[0], args.steps)
    _, incoming_ms = _timed(step.launches[-1], args.steps)
    torch.cuda.synchronize()
    diff = float((out2.float() - out.float()).abs().max())

    # prefetch one step ahead: steps alternate between the router's 16 nearest
    # chunks and the next 16; while a step runs, the other set (dropped from
    # its slots first, so that it really moves) is copied in without the
    # launch stream waiting, and the next step orders itself after the copy
    sets = [ids, router.rank(w.context - 1, w.context)[w.cold_attended:2 * w.cold_attended]]
    cache.evict_cold_slots()
    outs = [torch.empty_like(qd), torch.empty_like(qd)]
    launches = []
    for k in range(2):
        cache.prefetch_cold_chunks(sets[k])
        launches.append(cache.prepare(qd, causal=True, cold_chunks=sets[k], out=outs[k]))
        cache.note_reads(sets[k])  # the loop records each call's reads, so copies wait only for those
    slots_of = [sorted(cache.resident_cold_chunk(c)["slot"] for c in st) for st in sets]

    def ahead(i):
        cache.wait_for_prefetch()
        launches[i % 2]()
        cache.note_reads(sets[i % 2])
        nxt = sets[(i + 1) % 2]
        cache.evict_cold_slots(nxt)
        cache.prefetch_cold_chunks(nxt, wait=False)

    for i in range(args.warmup):
        ahead(i)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps (next step's chunks prefetched during the step)")
    t0 = time.perf_counter()
    for i in range(args.steps):
        ahead(i)
    cache.wait_for_prefetch()
    torch.cuda.synchronize()
    ahead_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    same_slots = slots_of == [sorted(cache.resident_cold_chunk(c)["slot"] for c in st) for st in sets]
    ahead_diff = float((outs[0].float() - out.float()).abs().max())

    step_bytes = w.bytes_per_step()
    achieved = step_bytes / (kernel_ms * 1e-3) / 1e9
    result = {
        "metric": "decode attn tokens/s + HBM GB/s (fused PQ+RVQ dequant-attn), 1 GPU",
        "value": round(w.batch / (ms_per_step * 1e-3), 1),
        "unit": "decode tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "warmup_run": warm,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) K/V with per-channel scale U(0.5,2); k-means codebooks on the warm span)",
        "config": {"workload": w.name, "batch": w.batch, "context": w.context, "q_heads": w.q_heads,
                   "kv_heads": w.kv_heads, "head_dim": w.head_dim, "hot_tokens": w.hot, "warm_tokens": w.warm,
                   "cold_tokens": w.cold, "cold_chunk_tokens": w.cold_chunk, "cold_chunks_attended": len(ids),
                   "cold_chunk_ids": ids,
                   "format": f"PQ M{w.pq_subspaces}x{w.pq_centroids} + RVQ M{w.rvq_subspaces}x{w.rvq_centroids}"
                             f" + top-{w.sparse_k} sparse (warm and cold)"},
        "hbm_gbs": round(achieved, 1),
        "bytes_per_step": step_bytes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(w.name),
                     "kernel_ms": round(kernel_ms, 5), "kernel_ms_percentiles": pct},
        "cold_copy_step": {
            "ms_per_step": round(refetch_ms, 5), "host_ms_per_step": round(refetch_host_ms, 5),
            "copy_bytes": step.copy_bytes, "copies": step.ncopies,
            "copy_ms": round(copy_ms, 5), "h2d_gbs": round(step.copy_bytes / (copy_ms * 1e-3) / 1e9, 2),
            "resident_part_ms": round(resident_ms, 5), "copied_part_ms": round(incoming_ms, 5),
            "tokens_per_s": round(w.batch / (refetch_ms * 1e-3), 1),
            "max_abs_vs_resident": diff},
        "prefetch_ahead_step": {
            "ms_per_step": round(ahead_ms, 5), "tokens_per_s": round(w.batch / (ahead_ms * 1e-3), 1),
            "copy_bytes_per_step": step.copy_bytes, "sets_kept_their_slots": same_slots,
            "max_abs_vs_resident": ahead_diff},
    }
    if not args.no_cpu:
        log("CPU baseline")
        result["cpu_baseline"], result["check_max_abs_vs_cpu"] = cpu_baseline_longctx(
            w, cache, ids, qd, out, args.cpu_repeats, budget_s=20.0 * args.cpu_budget)
    if args.stream_steps:
        result["stream"] = bench_stream(w, cache, router, (kq, vq), qd, args.stream_steps, dev)
    return result


def bench_stream(w, cache, router, quantizers, q, steps, dev) -> dict:
    """The decode loop's streaming path on the filled cache: each step appends
    one new token (hot ring; every 32 tokens a block is encoded into warm;
    whole chunks move from warm to pinned cold as warm fills), then attends
    hot + warm + the router's nearest cold chunks.  Wall-clock per step with
    the GPU synchronized at the end (the host issues everything)."""
    import torch
    from apple_amd.workloads import make_sequence

    kn, vn, _, _ = make_sequence(w, 1, tokens=3 * steps)
    kn, vn = kn.to(dev), vn.to(dev)
    chunks0, tok0 = len(cache.cold_chunk_metadata), cache.total_tokens
    log(f"streaming {steps} appends")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        cache.update(kn[i:i + 1], vn[i:i + 1], quantizers)
    torch.cuda.synchronize()
    append_ms = (time.perf_counter() - t0) * 1e3 / steps
    chunks1 = len(cache.cold_chunk_metadata)
    log(f"streaming {steps} decode steps (append + attention)")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps, 2 * steps):
        cache.update(kn[i:i + 1], vn[i:i + 1], quantizers)
        pos = cache.total_tokens - 1
        ids = router.rank(pos, cache.total_tokens)[:w.cold_attended]
        cache.attention_forward(q, causal=True, cold_chunks=ids)
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / steps
    # the same loop through a decode session: one prepared launch grown in
    # place while a step only adds a hot token and the chunk set stays
    sess = cache.decode_session(q, quantizers, router=router, cold_attended=w.cold_attended)
    sess.step(kn[2 * steps:2 * steps + 1], vn[2 * steps:2 * steps + 1])
    r0 = sess.rebuilds
    log(f"streaming {steps - 1} decode-session steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(2 * steps + 1, 3 * steps):
        sess.step(kn[i:i + 1], vn[i:i + 1])
    torch.cuda.synchronize()
    session_ms = (time.perf_counter() - t0) * 1e3 / (steps - 1)
    pos = cache.total_tokens - 1
    ref = cache.attention_forward(q, causal=True, cold_chunks=router.rank(pos, cache.total_tokens)[:w.cold_attended])
    return {"append_ms_per_token": round(append_ms, 4), "decode_step_ms": round(step_ms, 4),
            "decode_tokens_per_s": round(1e3 / step_ms, 1), "steps": steps,
            "session_step_ms": round(session_ms, 4), "session_tokens_per_s": round(1e3 / session_ms, 1),
            "session_rebuilds": sess.rebuilds - r0,
            "session_max_abs_vs_attention_forward": float((sess.out.float() - ref.float()).abs().max()),
            "tokens_appended": cache.total_tokens - tok0,
            "chunks_moved_to_cold": len(cache.cold_chunk_metadata) - chunks0,
            "chunks_moved_during_appends": chunks1 - chunks0,
            "tiers_after": {"hot": cache.num_hot, "warm": cache.num_warm, "cold": cache.num_cold}}


def cpu_baseline_longctx(w, cache, ids, q, gpu_out, repeats, budget_s=20.0):
    """The torch-CPU restatement over the same window: the chosen cold chunks
    and the warm tier decoded from their codes, then blockwise attention."""
    import torch
    from apple_amd.cache import _plain_head_major
    from oracle import cpu_baseline as cb

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    stores_k = [cache.load_cold_chunk(c)["key"] for c in sorted(ids)] + [cache.warm_keys]
    stores_v = [cache.load_cold_chunk(c)["value"] for c in sorted(ids)] + [cache.warm_values]
    codes = {}
    for kv, stores in (("k", stores_k), ("v", stores_v)):
        parts = [[None if t is None else t.cpu() for t in _plain_head_major(s)] for s in stores]
        codes[kv] = {name: torch.cat([p[i] for p in parts], 1)
                     for i, name in enumerate(("pq", "rvq", "sparse_idx", "sparse_val"))}
    cbs = {"k_pq": cache._kq.pq.codebooks.cpu(), "v_pq": cache._vq.pq.codebooks.cpu(),
           "k_rvq": cache._kq.rvq.codebooks.cpu(), "v_rvq": cache._vq.rvq.codebooks.cpu()}
    hk, hv = cache.hot_keys.permute(1, 0, 2).cpu(), cache.hot_values.permute(1, 0, 2).cpu()
    qc = q.cpu()
    out = cb.decode_step(qc, hk, hv, codes["k"], codes["v"], cbs, w.head_dim ** -0.5, w.block)  # warm-up
    n, t0 = 0, time.perf_counter()
    while n < repeats and time.perf_counter() - t0 < budget_s:
        out = cb.decode_step(qc, hk, hv, codes["k"], codes["v"], cbs, w.head_dim ** -0.5, w.block)
        n += 1
    sec = time.perf_counter() - t0
    err = float((out.float() - gpu_out.float().cpu()).abs().max())
    window = cache.num_hot + cache.num_warm + sum(min(w.cold_chunk, cache.num_cold - c * w.cold_chunk) for c in ids)
    return {"value": round(n / sec, 2), "unit": "decode tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} decode steps of the one sequence over the full {window}-token window "
                      f"(torch-CPU F.embedding decode of the {len(ids)} cold chunks + warm tier, fp32 "
                      f"blockwise attention, block {w.block})",
            "seconds": round(sec, 2)}, err


def traffic_from_profiles(workload: str, name: str = "fused_decode_attn_{}_traffic.md",
                          key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch (or step) measured by rocprofv3 PMC runs, if committed."""
    p = ROOT / "profiles" / name.format(workload)
    if not p.exists():
        return None
    m = re.search(key + r":\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the path shards by sequence with no "
                                   "communication, and multi-GPU runs are not part of it; use --gpus 1"}))
        return 2
    import torch

    if args.copy_calibration:
        print(json.dumps(copy_calibration(args.copy_calibration)), flush=True)
        return 0
    sys.path.insert(0, str(ROOT))
    from apple_amd.workloads import REF_WORKLOADS, WORKLOADS

    dev = torch.device("cuda", 0)
    if args.workload in REF_WORKLOADS:
        w = REF_WORKLOADS[args.workload]
        fn = bench_refencode if w.name.startswith("refencode") else bench_ref
        print(json.dumps(fn(w, args, dev)), flush=True)
        return 0
    w = WORKLOADS[args.workload]
    if w.name == "encode_4k":
        print(json.dumps(bench_encode(w, args, dev)), flush=True)
        return 0
    if w.cold:
        print(json.dumps(bench_longctx(w, args, dev)), flush=True)
        return 0
    if w.hot + w.warm != w.context or w.cold:
        raise SystemExit(f"workload {w.name} is not a hot+warm decode workload")
    log(f"workload {w.name}: B={w.batch} ctx={w.context} Hq={w.q_heads} Hkv={w.kv_heads} hot={w.hot} warm={w.warm}")
    cache, q = setup_decode(w, dev)
    out = torch.empty_like(q)
    launch = cache.prepare(q, splits=args.splits, out=out)
    warm = warm_up(launch, args.warmup)
    # HIP events on the launch stream bracket the timed region; the kernel
    # time per step is their interval over the K back-to-back launches
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        launch()
    end.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    kernel_ms = start.elapsed_time(end) / args.steps
    pct = step_percentiles(launch, args.steps)
    copy_gbs = device_copy_gbs()
    read_gbs = device_read_gbs()
    step_bytes = w.bytes_per_step()
    achieved = step_bytes / (kernel_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles(w.name)
    result = {
        "metric": "decode attn tokens/s + HBM GB/s (fused PQ+RVQ dequant-attn), 1 GPU",
        "value": round(w.batch / (ms_per_step * 1e-3), 1),
        "unit": "decode tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_run": warm,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) K/V with per-channel scale U(0.5,2); k-means codebooks per sequence)",
        "config": {"workload": w.name, "batch": w.batch, "context": w.context, "q_heads": w.q_heads,
                   "kv_heads": w.kv_heads, "head_dim": w.head_dim, "hot_tokens": w.hot, "warm_tokens": w.warm,
                   "format": f"PQ M{w.pq_subspaces}x{w.pq_centroids}"
                             + (f" + RVQ M{w.rvq_subspaces}x{w.rvq_centroids}" if w.rvq_subspaces else "")
                             + (f" + top-{w.sparse_k} sparse" if w.sparse_k else ""),
                   "k_scoring": launch.k_scoring},
        "hbm_gbs": round(achieved, 1),
        "bytes_per_step": step_bytes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel_ms": round(kernel_ms, 5), "kernel_ms_percentiles": pct,
                     "device_copy_gbs": copy_gbs, "frac_of_device_copy": round(achieved / copy_gbs, 4),
                     "device_read_gbs": read_gbs, "frac_of_device_read": round(achieved / read_gbs, 4)},
    }
    if cache.last_drift is not None and cache.k_layout == 1 and launch.k_scoring == "fp16 q.centroid tables":
        # drift [B, Hq, splits]; a block (sequence, KV head, split) recomputes when one of its heads fires
        tol = cache.config.score_table_tolerance
        d = cache.last_drift.float().view(w.batch, w.kv_heads, w.q_heads // w.kv_heads, -1)
        result["score_table_guard"] = {"tolerance": tol, "drift_max": float(d.max()),
                                       "blocks_recomputed": int((d.amax(2) > tol).sum()),
                                       "blocks": int(d.amax(2).numel())}
    if cache.k_layout == 1 and not args.no_exact:
        log("exact codebook K path")
        result["exact_k_path"] = exact_path(w, cache, q, out, args.steps, dev)
    if not args.no_cpu:
        log("CPU baseline")
        cpu, err = cpu_baseline(w, cache, q, out, args.cpu_sample, args.cpu_repeats)
        four, _ = cpu_baseline(w, cache, q, out, args.cpu_sample, max(4, args.cpu_repeats // 4), threads=4)
        cpu["at_4_threads"] = {k: four[k] for k in ("value", "cores", "seconds")}
        result["cpu_baseline"] = cpu
        result["check_max_abs_vs_cpu"] = err
    if w.name == "batched_32x32k" and not args.no_extras:
        # the encode and long-context workloads timed in the same run, after
        # the headline's timed region (shorter warm-ups and CPU budgets)
        del cache, launch
        torch.cuda.empty_cache()
        sub = argparse.Namespace(**dict(vars(args), warmup=100, steps=256, splits=0, cpu_budget=0.4,
                                        stream_steps=300, cpu_repeats=16))
        log("sub-record encode_4k")
        result["encode_4k"] = sub_record(bench_encode(WORKLOADS["encode_4k"], sub, dev))
        log("sub-record longctx_128k")
        result["longctx_128k"] = sub_record(bench_longctx(WORKLOADS["longctx_128k"], sub, dev))
        log("sub-record refencode_4k")
        result["refencode_4k"] = sub_record(bench_refencode(REF_WORKLOADS["refencode_4k"], sub, dev))
        log("sub-record refdefault_32k")
        result["refdefault_32k"] = sub_record(bench_ref(REF_WORKLOADS["refdefault_32k"], sub, dev))
    print(json.dumps(result), flush=True)
    return 0


def sub_record(r: dict) -> dict:
    """A workload's line without the keys the headline line already states."""
    drop = ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline", "data", "warmup_run")
    out = {k: v for k, v in r.items() if k not in drop}
    out["metric"] = r["metric"]
    return out


if __name__ == "__main__":
    sys.exit(main())
