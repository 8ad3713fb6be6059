#!/usr/bin/env python3
"""Decode-attention + KV-append throughput on one MI355X (Qwen3-4B shape).

One step = one decode step of a 36-layer Qwen3-4B-shaped model's KV path:
for every layer, append one new token per sequence into that layer's paged
cache (slot-mapped) and run GQA paged decode attention over the full context.
Shape: batch 64, context 4096 (4095 cached + the new token), 32 query / 8 KV
heads, head_dim 128, bf16 KV, block 16. Every layer has its own 1 GiB cache
(36 GiB in total, far beyond the 256 MB Infinity Cache), so consecutive
layers never hit in cache. Inputs are synthetic and already resident in HBM.

Prints one JSON line:
  value        algorithmic bytes of a step / measured step time (GB/s)
  roofline     one layer's fused append + attention launch: algorithmic bytes
               per launch / its mean time (HIP events on the launch stream),
               against the 8 TB/s HBM peak
  cpu_baseline the CPU oracle on a bounded sample of the same workload
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--partition", type=int, default=0, help="tokens per split-K partition (0 = library choice)")
    ap.add_argument("--kernel-reps", type=int, default=2, help="passes over all layers for per-launch timing")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU oracle time budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy 1 GiB device to device (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def calibrate_copy() -> int:
    """One plain 1 GiB device-to-device copy: reads 1 GiB and writes 1 GiB of HBM."""
    import torch

    a = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copied_bytes": a.numel() * 4}))
    return 0


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_gqa_qwen3_4b_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch") and kernel in line:
                    return int(line.split()[1])
    except OSError:
        pass
    return None


def algorithmic_bytes(batch: int, context: int, hq: int, hkv: int, d: int, bs: int, kv_bytes: int = 2) -> dict:
    """Per-layer bytes of the KV path, as the path must move them at minimum."""
    kv = batch * context * 2 * hkv * d * kv_bytes  # K and V of every context token
    qo = batch * hq * d * 2 * 2  # q in, o out (bf16)
    bt = batch * ((context + bs - 1) // bs) * 4  # block-table entries read
    sl = batch * 4  # seq_lens
    attn = kv + qo + bt + sl
    append = batch * 2 * hkv * d * (2 + kv_bytes) + batch * 8  # new K/V in + cache write + slots
    return {"attention": attn, "append": append, "layer": attn + append}


def cpu_baseline(args, hq, hkv, d, bs, scale, per_layer_bytes) -> dict:
    """The oracle (numpy) on a bounded sample: one layer of a few sequences, append + attention."""
    from oracle import paged
    from wavelet_amd import synth

    try:
        from threadpoolctl import threadpool_info, threadpool_limits

        cores = len(os.sched_getaffinity(0))
        limiter = threadpool_limits(limits=cores)
        blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        cores = blas[0]["num_threads"] if blas else cores
    except Exception:  # threadpoolctl missing: whatever numpy uses
        limiter, cores = None, len(os.sched_getaffinity(0))
    nseq = 4
    w = synth.make_decode_workload("cpu-sample", batch=nseq, num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=bs, context_lens=np.full(nseq, args.context))
    kc, vc = paged.empty_cache(w.num_blocks, bs, hkv, d)
    kc[...] = synth.normal_bf16(synth.stream_key("cpu-sample", "k"), kc.shape)
    vc[...] = synth.normal_bf16(synth.stream_key("cpu-sample", "v"), vc.shape)
    q = paged.bf16_to_f32(synth.normal_bf16(synth.stream_key("cpu-sample", "q"), (nseq, hq, d)))
    kn = synth.normal_bf16(synth.stream_key("cpu-sample", "kn"), (nseq, hkv, d))
    vn = synth.normal_bf16(synth.stream_key("cpu-sample", "vn"), (nseq, hkv, d))
    slots = w.new_token_slots()

    def one_layer():
        paged.append_bf16(kc, vc, kn, vn, slots)
        gk, gv = paged.gather(kc, vc, w.block_tables, w.context_lens)
        kf = paged.bf16_to_f32(gk).reshape(nseq, args.context, hkv, d)
        vf = paged.bf16_to_f32(gv).reshape(nseq, args.context, hkv, d)
        g = hq // hkv
        for i in range(nseq):
            for h in range(hkv):
                s = (q[i, h * g:(h + 1) * g] @ kf[i, :, h].T) * np.float32(scale)
                s = np.exp(s - s.max(axis=1, keepdims=True))
                s /= s.sum(axis=1, keepdims=True)
                _ = s @ vf[i, :, h]

    one_layer()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        one_layer()
        reps += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or reps >= 1000:
            break
    if limiter is not None:
        limiter.unregister() if hasattr(limiter, "unregister") else None
    sample_bytes = per_layer_bytes * nseq / args.batch
    return {
        "value": round(sample_bytes * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": int(cores),
        "kind": "port",
        "sample": f"{reps} x (one layer, {nseq} of the {args.batch} sequences: append 1 token + attention over "
                  f"{args.context} tokens), {el:.1f} s, numpy oracle",
    }


def main() -> int:
    args = parse()
    if args.calibrate_copy:
        return calibrate_copy()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); run it with --gpus 1", file=sys.stderr)
        return 2
    import torch

    from wavelet_amd import PagedKVCache, synth
    from wavelet_amd.plan import DecodeStep

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, L, HQ, HKV, D, BS = args.batch, args.context, 32, 8, 128, 16
    scale = 1.0 / np.sqrt(D)
    nb = B * ((L + BS - 1) // BS)
    w = synth.make_decode_workload("bench-qwen3-4b", batch=B, num_kv_heads=HKV, num_q_heads=HQ, head_dim=D,
                                   block_size=BS, context_lens=np.full(B, L), num_blocks=nb)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    caches, qs, ks, vs, outs = [], [], [], [], []
    for _ in range(args.layers):
        c = PagedKVCache(nb, BS, HKV, D, device=dev)
        c.k.normal_(generator=gen)
        c.v.normal_(generator=gen)
        caches.append(c)
        qs.append(torch.randn((B, HQ, D), generator=gen, device=dev).to(torch.bfloat16))
        ks.append(torch.randn((B, HKV, D), generator=gen, device=dev).to(torch.bfloat16))
        vs.append(torch.randn((B, HKV, D), generator=gen, device=dev).to(torch.bfloat16))
        outs.append(torch.empty((B, HQ, D), dtype=torch.bfloat16, device=dev))
    bt = torch.from_numpy(w.block_tables).to(dev)
    sl = torch.from_numpy(w.context_lens).to(dev)
    slots = torch.from_numpy(w.new_token_slots()).to(dev)
    step = DecodeStep(caches, qs, ks, vs, outs, bt, sl, slots, scale, max_seq_len=L, partition_size=args.partition)
    torch.cuda.synchronize()
    print(f"# setup done: {args.layers} layers x {caches[0].nbytes / 2**30:.2f} GiB cache", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        step.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step.run()
    e1.record()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall
    ms_per_step = e0.elapsed_time(e1) / args.steps
    print(f"# timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step (wall {t_wall / args.steps * 1e3:.2f} ms/step)",
          file=sys.stderr, flush=True)

    # Per-launch timing of one layer's fused append + attention (the decode
    # kernel and, when a context spans several partitions, its merge kernel),
    # layer caches rotated so no layer is re-read from cache.
    def per_launch(fn, reps):
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(reps * args.layers)]
        i = 0
        for _ in range(reps):
            for layer in range(args.layers):
                a, b = pairs[i]
                a.record()
                fn(layer)
                b.record()
                i += 1
        torch.cuda.synchronize()
        return float(np.mean([a.elapsed_time(b) for a, b in pairs])) * 1e3

    kernel_us = per_launch(step.step_layer, args.kernel_reps)
    attend_us = per_launch(step.attend, 1)
    append_us = per_launch(step.append, 1)

    by = algorithmic_bytes(B, L, HQ, HKV, D, BS)
    step_bytes = by["layer"] * args.layers
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = by["layer"] / (kernel_us * 1e-6) / 1e9
    rec = {
        "metric": "decode-attn+KV-append GB/s (% of HBM peak) & us/step, Qwen3-4B B=64 4k ctx",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "us_per_step": round(ms_per_step * 1e3, 1),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random bf16 K/V/q, seeded), resident in HBM",
        "config": {
            "workload": "Qwen3-4B decode step: 36 layers x (append 1 token/seq + GQA paged decode attention)",
            "layers": args.layers, "batch": B, "context": L, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
            "block_size": BS, "kv_dtype": "bf16", "partition_size": args.partition or "auto",
            "bytes_per_step": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_gqa_kernel<128,false,true,4>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("decode_gqa_kernel<128,false,true,4>"),
            "bytes_per_launch": by["layer"],
            "mean_launch_us": round(kernel_us, 2),
        },
        "unfused_us": {"append": round(append_us, 2), "attention": round(attend_us, 2)},
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline(args, HQ, HKV, D, BS, scale, by["layer"])
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
