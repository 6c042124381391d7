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
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="batched_32x32k")
    ap.add_argument("--splits", type=int, default=0, help="token splits per (sequence, KV head); 0 = auto")
    ap.add_argument("--cpu-sample", type=int, default=4, help="sequences timed on the CPU baseline")
    ap.add_argument("--cpu-repeats", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    return ap.parse_args(argv)


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


def cpu_baseline(w, cache, q, gpu_out, sample, repeats):
    """Time the torch-CPU restatement of the path on a bounded sample."""
    import torch
    from apple_amd.batched import untile
    from oracle import cpu_baseline as cb

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    f = cache.fmt
    total, n, max_err = 0.0, 0, 0.0
    for b in range(min(sample, w.batch)):
        nw, nh = cache.num_warm[b], cache.num_hot[b]
        codes = {}
        for kv in ("k", "v"):
            c = cache.codes[kv]
            codes[kv] = {"pq": untile(c["pq"][b], f.pq_subspaces, nw).cpu()}
            if f.rvq_subspaces:
                codes[kv]["rvq"] = untile(c["rvq"][b], f.rvq_subspaces, nw).cpu()
            if f.sparse_k:
                codes[kv]["sparse_idx"] = c["sparse_idx"][b, :, :nw].cpu()
                codes[kv]["sparse_val"] = c["sparse_val"][b, :, :nw].cpu()
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

    def step():
        for (x, _), (pcb, rcb) in zip(xs, cbs):
            K.warm_encode(x, fmt, pcb, rcb)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"timing {args.steps} encode steps")
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    kernel_ms = start.elapsed_time(end) / args.steps
    vectors = 2 * w.context * w.kv_heads
    # algorithmic contraction flops: 2 * C * D per vector and stage
    flops = vectors * 2 * w.head_dim * (w.pq_centroids + (w.rvq_centroids if w.rvq_subspaces else 0))
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    result = {
        "metric": "warm-tier encode vectors/s (PQ+RVQ+top-k, MFMA nearest-centroid search), 1 GPU",
        "value": round(vectors / (kernel_ms * 1e-3), 1),
        "unit": "vectors/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
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
                     "flops_per_step": flops},
    }
    if not args.no_cpu:
        log("CPU baseline")
        from oracle import numerics as nx

        n = min(args.cpu_sample * 512, w.context * w.kv_heads)
        x = xs[0][0][:n].cpu().numpy()
        pcb, rcb = (t.cpu().numpy() if t is not None else None for t in cbs[0])
        t0 = time.perf_counter()
        nx.ext_encode(x, pcb, rcb, fmt.sparse_k)
        sec = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(n / sec, 1), "unit": "vectors/s", "cores": 1, "kind": "port",
                                  "sample": f"{n} key vectors of the chunk through the oracle's numpy encode "
                                            f"(float64 brute-force distances), one process",
                                  "seconds": round(sec, 2)}
    return result


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs, if committed."""
    p = ROOT / "profiles" / f"fused_decode_attn_{workload}_traffic.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
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
    from apple_amd.workloads import WORKLOADS

    w = WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    if w.name == "encode_4k":
        print(json.dumps(bench_encode(w, args, dev)), flush=True)
        return 0
    if w.hot + w.warm != w.context or w.cold:
        raise SystemExit(f"workload {w.name} is not a hot+warm decode workload")
    log(f"workload {w.name}: B={w.batch} ctx={w.context} Hq={w.q_heads} Hkv={w.kv_heads} hot={w.hot} warm={w.warm}")
    cache, q = setup_decode(w, dev)
    out = torch.empty_like(q)
    launch = cache.prepare(q, splits=args.splits, out=out)
    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
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
                             + (f" + top-{w.sparse_k} sparse" if w.sparse_k else "")},
        "hbm_gbs": round(achieved, 1),
        "bytes_per_step": step_bytes,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel_ms": round(kernel_ms, 5)},
    }
    if not args.no_cpu:
        log("CPU baseline")
        cpu, err = cpu_baseline(w, cache, q, out, args.cpu_sample, args.cpu_repeats)
        result["cpu_baseline"] = cpu
        result["check_max_abs_vs_cpu"] = err
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
