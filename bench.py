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
               against the 8 TB/s HBM peak; `traffic` is the HBM bytes per
               launch from the committed rocprofv3 PMC summary named in
               `traffic_source` (counters cannot be read inside this run)
  hbm_read_ceiling_gbs  a read-only streaming kernel over 4 GiB, same process
  cpu_baseline the numpy oracle on a bounded sample of the same workload:
               median of >= 5 timed repetitions after one warm-up
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
NO_KV_DTYPE = ("deepseek-v3-mla", "sampler", "sampler-default")  # workloads without a GQA KV cache
MFMA_PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="qwen3-4b",
                    choices=["qwen3-4b", "qwen3-4b-var", "qwen2.5-0.5b", "qwen2.5-7b-groups", "deepseek-v3-mla",
                             "qwen3-4b-prefill", "sampler", "sampler-default"],
                    help="qwen3-4b is the headline; the others are the remaining measured shapes")
    ap.add_argument("--layers", type=int, default=0, help="0 = the model's depth (8 rotated layers for MLA)")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--kv-dtype", default=None, choices=["bf16", "fp8_e4m3"],
                    help="KV cache dtype of a GQA workload (default: bf16, fp8_e4m3 for qwen2.5-7b-groups); "
                         "the MLA and sampler workloads have none")
    ap.add_argument("--partition", type=int, default=0, help="tokens per split-K partition (0 = library choice)")
    ap.add_argument("--kernel-reps", type=int, default=2, help="passes over all layers for per-launch timing")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU oracle time budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--plain-decode", action="store_true",
                    help="qwen2.5-7b-groups: decode every member with the plain call (shared prompt blocks and "
                         "private tokens read with one policy, batch-wide longest-first order) instead of the "
                         "group-aware decode, the default")
    ap.add_argument("--via-pool", action="store_true",
                    help="qwen3-4b / qwen3-4b-var: build the caches as the engine does -- a KVPool sized by "
                         "KVPool.from_engine_config (gpu_memory_utilization 0.35), tables and slots from its block "
                         "manager, each step's read policy from the manager's reference counts")
    ap.add_argument("--graph", action="store_true",
                    help="GQA decode workloads (not the group-aware qwen2.5-7b-groups default): time replays of the whole step captured in one "
                         "HIP graph (GraphDecodeStep, the allocation-free entry point) instead of eager launches; "
                         "the eager step time is reported beside it")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy 1 GiB device to device (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--phase-clocks", action="store_true",
                    help="deepseek-v3-mla only: run the attention with the profiling library "
                         "(python -m wavelet_amd.build --phase-clocks) and print its per-phase cycle counts")
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


def hbm_read_ceiling_gbs(torch, dev, nbytes: int = 4 << 30, reps: int = 5) -> dict:
    """Best read rate of the library's streaming-read probe over a 4 GiB buffer (16x the
    256 MB last-level cache), a few grid sizes, HIP events on the launch stream."""
    from wavelet_amd import _lib

    lib = _lib.load()
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    buf.fill_(0x5A)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    best, best_blocks = 0.0, 0
    for blocks in (2048, 4096, 8192, 16384):
        rc = lib.wkv_hbm_read_probe(buf.data_ptr(), nbytes, blocks, sink.data_ptr(), stream.cuda_stream)
        _lib.check(rc, "hbm read probe")
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            lib.wkv_hbm_read_probe(buf.data_ptr(), nbytes, blocks, sink.data_ptr(), stream.cuda_stream)
        b.record(stream)
        torch.cuda.synchronize()
        gbs = nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9
        if gbs > best:
            best, best_blocks = gbs, blocks
    del buf, sink
    torch.cuda.empty_cache()
    return {"gbs": round(best, 1), "bytes": nbytes, "workgroups": best_blocks}


# committed rocprofv3 PMC summaries per workload (bf16 KV unless named)
TRAFFIC_PROFILES = {
    ("qwen3-4b", "bf16"): "profiles/decode_gqa_qwen3_4b_pmc.md",
    ("qwen3-4b-var", "bf16"): "profiles/decode_gqa_qwen3_4b_var_pmc.md",
    ("qwen2.5-0.5b", "bf16"): "profiles/decode_gqa_qwen2_5_0_5b_pmc.md",
    ("deepseek-v3-mla", "bf16"): "profiles/decode_mla_deepseek_v3.md",
    ("qwen2.5-7b-groups", "fp8_e4m3"): "profiles/decode_gqa_fp8_groups.md",
}


def measured_traffic(workload: str, kv_dtype: str, kernel: str) -> tuple[int | None, str | None]:
    """HBM bytes per launch of `kernel` from the workload's committed rocprofv3 PMC summary,
    and where that figure comes from (the summary file and the commit it records), if any."""
    rel = TRAFFIC_PROFILES.get((workload, kv_dtype))
    if rel is None:
        return None, None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), rel)
    value, commit = None, None
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch") and kernel in line:
                    value = int(line.split()[1])
                elif line.startswith("source_commit"):
                    commit = line.split()[1]
    except OSError:
        return None, None
    if value is None:
        return None, None
    src = f"{rel}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this workload"
    return value, src + (f" at commit {commit}" if commit else "")


def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


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

    one_layer()  # warm-up, untimed
    times, t0 = [], time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t0 < args.cpu_seconds and len(times) < 1000):
        t = time.perf_counter()
        one_layer()
        times.append(time.perf_counter() - t)
    if limiter is not None:
        limiter.unregister() if hasattr(limiter, "unregister") else None
    sample_bytes = per_layer_bytes * nseq / args.batch
    med = float(np.median(times))
    return {
        "value": round(sample_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": int(cores),
        "kind": "port",
        "impl": "numpy restatement of the path (oracle/paged.py: append_bf16, gather, fp32 attention), "
                "BLAS threads = cores",
        "cpu_model": cpu_model(),
        "reps": len(times),
        "median_s": round(med, 4),
        "sample": f"median of {len(times)} timed reps after 1 warm-up of (one layer, {nseq} of the {args.batch} "
                  f"sequences: append 1 token + attention over {args.context} tokens), "
                  f"{sum(times):.1f} s in total; GB/s = that sample's algorithmic bytes / median time",
    }


def gqa_cache(w, kv_dtype: str, dev):
    """One layer's cache for a GQA workload, as every GQA workload builds it (the parity tests
    of the benchmarked plans build theirs through this same call): a workload whose groups share
    prompt blocks says so, and its decodes then keep shared blocks cached."""
    from wavelet_amd import PagedKVCache

    return PagedKVCache(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, kv_dtype=kv_dtype, device=dev,
                        shared_blocks=w.group_size > 1)


def _gqa_setup(torch, dev, args, w, kv_dtype: str, qkv_std: float = 1.0, grouped: bool = False):
    """Per-layer caches (own memory per layer), step buffers and a DecodeStep plan
    (group-aware when `grouped`: the workload's groups share their prompt blocks)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    B, HQ, HKV, D, BS = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size
    caches, qs, ks, vs, outs = [], [], [], [], []
    for _ in range(args.layers):
        c = gqa_cache(w, kv_dtype, dev)
        if kv_dtype == "bf16":
            c.k.normal_(generator=gen)
            c.v.normal_(generator=gen)
            if qkv_std != 1.0:
                c.k.mul_(qkv_std)
                c.v.mul_(qkv_std)
        else:  # random finite e4m3 codes (no 0x7F/0xFF NaN codes) and power-of-two scales
            for t in (c.k, c.v):
                t.copy_(torch.randint(0, 256, t.shape, generator=gen, device=dev, dtype=torch.int32)
                        .to(torch.uint8) & 0xF7)
            c.k_scale.fill_(2.0 ** -8)
            c.v_scale.fill_(2.0 ** -8)
        caches.append(c)
        qs.append((torch.randn((B, HQ, D), generator=gen, device=dev) * qkv_std).to(torch.bfloat16))
        ks.append((torch.randn((B, HKV, D), generator=gen, device=dev) * qkv_std).to(torch.bfloat16))
        vs.append((torch.randn((B, HKV, D), generator=gen, device=dev) * qkv_std).to(torch.bfloat16))
        outs.append(torch.empty((B, HQ, D), dtype=torch.bfloat16, device=dev))
    step = gqa_plan(torch, dev, w, caches, qs, ks, vs, outs, args.partition, grouped)
    return step, caches[0].nbytes


class _StepWithPolicy:
    """A DecodeStep launched with one read policy for every step (the policy a serving loop
    computes per step; fixed here because the benchmark's tables do not change)."""

    grouped = False

    def __init__(self, step, shared_blocks: bool) -> None:
        self.step, self.shared_blocks = step, bool(shared_blocks)

    def run(self) -> None:
        self.step.run(shared_blocks=self.shared_blocks)

    def step_layer(self, layer: int) -> None:
        self.step.step_layer(layer, self.shared_blocks)

    def attend(self, layer: int) -> None:
        self.step.attend(layer, self.shared_blocks)

    def append(self, layer: int) -> None:
        self.step.append(layer)


def _gqa_pool_setup(torch, dev, args, w, kv_dtype: str):
    """The workload through the engine-facing surface: one KVPool sized by
    KVPool.from_engine_config (the engine's default gpu_memory_utilization 0.35,
    max_model_len = the longest context), every sequence's cached context allocated by the
    pool's block manager (distinct salts: nothing shared), the step's slots from
    KVPool.append_slots and its tables from the manager, and the read policy from the
    manager's reference counts (KVPool.decode_shares_blocks). Returns the step, the cache
    bytes per layer, and the workload with the manager's tables."""
    import dataclasses

    from wavelet_amd import KVPool
    from wavelet_amd.plan import DecodeStep

    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    B, HQ, HKV, D, BS = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size
    L = w.context_lens.astype(np.int64)
    pool = KVPool.from_engine_config(num_layers=args.layers, num_kv_heads=HKV, head_dim=D, kv_dtype=kv_dtype,
                                     block_size=BS, gpu_memory_utilization=0.35, max_model_len=int(L.max()),
                                     device=dev)
    ids = list(range(B))
    for i in ids:
        pool.blocks.allocate(i, np.arange(int(L[i]) - 1), cache_salt=f"seq{i}")
    slots = pool.append_slots(ids)
    bt, lens = pool.blocks.tables(ids)
    n_used = int(bt.max()) + 1
    qs, ks, vs, outs = [], [], [], []
    for c in pool.layers:
        if kv_dtype == "bf16":
            c.k[:n_used].normal_(generator=gen)
            c.v[:n_used].normal_(generator=gen)
        else:
            for t in (c.k, c.v):
                t[:n_used].copy_(torch.randint(0, 256, t[:n_used].shape, generator=gen, device=dev,
                                               dtype=torch.int32).to(torch.uint8) & 0xF7)
            c.k_scale.fill_(2.0 ** -8)
            c.v_scale.fill_(2.0 ** -8)
        qs.append(torch.randn((B, HQ, D), generator=gen, device=dev).to(torch.bfloat16))
        ks.append(torch.randn((B, HKV, D), generator=gen, device=dev).to(torch.bfloat16))
        vs.append(torch.randn((B, HKV, D), generator=gen, device=dev).to(torch.bfloat16))
        outs.append(torch.empty((B, HQ, D), dtype=torch.bfloat16, device=dev))
    step = DecodeStep(pool.layers, qs, ks, vs, outs, torch.from_numpy(bt).to(dev), torch.from_numpy(lens).to(dev),
                      slots, w.scale, max_seq_len=int(lens.max()), partition_size=args.partition)
    shared = pool.decode_shares_blocks(ids)
    w2 = dataclasses.replace(w, num_blocks=pool.num_blocks, block_tables=bt,
                             context_lens=lens.astype(w.context_lens.dtype))
    return _StepWithPolicy(step, shared), pool.nbytes // args.layers, w2, pool


def gqa_plan(torch, dev, w, caches, qs, ks, vs, outs, partition: int = 0, grouped: bool = False):
    """The decode plan every GQA workload times: fused append + attention per layer, the
    library's partition and dispatch order unless `partition` is given, group-aware when
    `grouped` (the parity tests build their plans through this same call)."""
    from wavelet_amd.plan import DecodeStep

    bt = torch.from_numpy(w.block_tables).to(dev)
    sl = torch.from_numpy(w.context_lens).to(dev)
    slots = torch.from_numpy(w.new_token_slots()).to(dev)
    group = {}
    if grouped:
        n_groups = w.batch // w.group_size
        group = dict(group_size=w.group_size, max_prefix_len=w.prefix_len,
                     prefix_lens=torch.full((n_groups,), w.prefix_len, dtype=torch.int32, device=dev))
    return DecodeStep(caches, qs, ks, vs, outs, bt, sl, slots, w.scale, max_seq_len=int(w.context_lens.max()),
                      partition_size=partition, **group)


def mla_plan(torch, dev, w, caches, q_nope, q_pe, kv_c, k_pe, outs, partition: int = 0):
    """The MLA decode plan the deepseek-v3-mla workload times (fused latent append + attention)."""
    from wavelet_amd.plan import MLADecodeStep

    return MLADecodeStep(caches, q_nope, q_pe, kv_c, k_pe, outs, torch.from_numpy(w.block_tables).to(dev),
                         torch.from_numpy(w.context_lens).to(dev), torch.from_numpy(w.new_token_slots()).to(dev),
                         w.scale, max_seq_len=int(w.context_lens.max()), partition_size=partition)


def workload(args, torch, dev) -> dict:
    """Builds the selected workload: plan, bytes, names (the default is the headline)."""
    from wavelet_amd import MLALatentCache, synth

    name = args.workload
    kv_dtype = getattr(args, "kv_dtype", None)
    stream = None  # the decode's read policy, when the step chooses it
    if name in ("qwen3-4b", "qwen3-4b-var"):
        w = synth.qwen3_4b_workload(batch=args.batch, context=args.context if name == "qwen3-4b" else None)
        args.layers = args.layers or 36
        kv_dtype = kv_dtype or "bf16"
        desc = f"Qwen3-4B decode step: 36 layers x (append 1 token/seq + GQA paged decode attention), {kv_dtype} KV"
        if getattr(args, "via_pool", False):
            step, cache_bytes, w, _pool = _gqa_pool_setup(torch, dev, args, w, kv_dtype)
            stream = not step.shared_blocks
            desc += (", through KVPool.from_engine_config(gpu_memory_utilization=0.35) with block-manager tables "
                     f"and the per-step read policy ({'streamed' if stream else 'cached'})")
        else:
            step, cache_bytes = _gqa_setup(torch, dev, args, w, kv_dtype)
        kv_bytes = 1 if kv_dtype == "fp8_e4m3" else 2
    elif getattr(args, "via_pool", False):
        raise SystemExit("--via-pool applies to the qwen3-4b and qwen3-4b-var workloads")
    elif name == "qwen2.5-0.5b":
        w = synth.qwen25_05b_workload()
        args.layers = args.layers or 24
        kv_dtype = kv_dtype or "bf16"
        step, cache_bytes = _gqa_setup(torch, dev, args, w, kv_dtype, qkv_std=1 / 8)
        kv_bytes = 1 if kv_dtype == "fp8_e4m3" else 2
        desc = f"Qwen2.5-0.5B decode step: 24 layers x (append + GQA decode), 14 q / 2 kv heads, d=64, {kv_dtype} KV"
    elif name == "qwen2.5-7b-groups":
        w = synth.qwen25_7b_group_workload()
        args.layers = args.layers or 28
        grouped = not getattr(args, "plain_decode", False)
        kv_dtype = kv_dtype or "fp8_e4m3"
        step, cache_bytes = _gqa_setup(torch, dev, args, w, kv_dtype, grouped=grouped)
        kv_bytes = 1 if kv_dtype == "fp8_e4m3" else 2
        desc = (f"Qwen2.5-7B GRPO groups, {kv_dtype} KV: 28 layers x (append + GQA decode), 32 x 8 seqs, shared "
                "1024-token prompts" + (" (group-aware: prompt blocks cached, members' own tokens streamed, "
                                        "a group's members on one XCD)" if grouped else
                                        " (members decoded separately)"))
    elif name == "deepseek-v3-mla":
        w = synth.deepseek_v3_mla_workload()
        args.layers = args.layers or 8
        gen = torch.Generator(device=dev)
        gen.manual_seed(1234)
        B, H, R, P, BS = w.batch, w.num_q_heads, 512, 64, w.block_size
        caches, qn, qp, kc, kp, outs = [], [], [], [], [], []
        for _ in range(args.layers):
            c = MLALatentCache(w.num_blocks, BS, R, P, device=dev)
            c.latent.normal_(generator=gen)
            caches.append(c)
            qn.append(torch.randn((B, H, R), generator=gen, device=dev).to(torch.bfloat16))
            qp.append(torch.randn((B, H, P), generator=gen, device=dev).to(torch.bfloat16))
            kc.append(torch.randn((B, R), generator=gen, device=dev).to(torch.bfloat16))
            kp.append(torch.randn((B, P), generator=gen, device=dev).to(torch.bfloat16))
            outs.append(torch.empty((B, H, R), dtype=torch.bfloat16, device=dev))
        step = mla_plan(torch, dev, w, caches, qn, qp, kc, kp, outs, args.partition)
        cache_bytes = caches[0].latent.numel() * 2
        L = w.context_lens.astype(np.int64)
        attn = int(L.sum()) * (R + P) * 2 + B * H * (R + P) * 2 + B * H * R * 2 + int(((L + BS - 1) // BS).sum()) * 4 + B * 4
        append = B * (R + P) * 2 * 2 + B * 8
        flops = 2 * int(L.sum()) * H * (R + P + R)
        return {"name": name, "step": step, "w": w, "layer_bytes": attn + append, "attn_bytes": attn,
                "kernel": "decode_mla_kernel<4> x2 head groups (+ mla_merge_kernel)", "dtype": "bf16", "kv_dtype": "bf16",
                "flops_per_layer": flops,
                "cache_bytes": cache_bytes,
                "desc": f"DeepSeek-V3 MLA decode: {args.layers} layers x (latent append + absorbed attention), "
                        "128 heads, 512+64 latent, B=32, context 4096, block 64"}
    elif name == "qwen3-4b-prefill":
        # the prompt step: 8 prompts of 2,048 tokens, no cached context
        from wavelet_amd import PagedKVCache
        from wavelet_amd.plan import PrefillStep

        n_new, B = 2048, 8
        kv_dtype = kv_dtype or "bf16"
        w = synth.make_decode_workload(name, batch=B, num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                                       context_lens=np.full(B, n_new))
        args.layers = args.layers or 36
        gen = torch.Generator(device=dev)
        gen.manual_seed(1234)
        T, HQ, HKV, D, BS = B * n_new, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size
        caches, qs, ks, vs, outs = [], [], [], [], []
        for _ in range(args.layers):
            caches.append(PagedKVCache(w.num_blocks, BS, HKV, D, kv_dtype=kv_dtype, device=dev))
            qs.append(torch.randn((T, HQ, D), generator=gen, device=dev).to(torch.bfloat16))
            ks.append(torch.randn((T, HKV, D), generator=gen, device=dev).to(torch.bfloat16))
            vs.append(torch.randn((T, HKV, D), generator=gen, device=dev).to(torch.bfloat16))
            outs.append(torch.empty((T, HQ, D), dtype=torch.bfloat16, device=dev))
        pos = np.arange(n_new)
        slots = np.concatenate([w.block_tables[i][pos // BS].astype(np.int64) * BS + pos % BS for i in range(B)])
        cu = torch.arange(0, T + 1, n_new, dtype=torch.int32, device=dev)
        step = PrefillStep(caches, qs, ks, vs, outs, torch.from_numpy(w.block_tables).to(dev),
                           torch.from_numpy(w.context_lens).to(dev), cu, torch.from_numpy(slots).to(dev), w.scale,
                           max_query_len=n_new, max_seq_len=n_new)
        visible = B * n_new * (n_new + 1) // 2  # (query, key) pairs under the causal mask
        flops = 4 * visible * HQ * D
        fp8 = kv_dtype == "fp8_e4m3"
        kvb = 1 if fp8 else 2  # cache bytes per element
        append = T * 2 * HKV * D * (2 + kvb) + T * 8
        attn = T * HQ * D * 2 * 2 + T * 2 * HKV * D * kvb  # q in, o out, the prompt's K/V read once
        return {"name": name, "step": step, "w": w, "layer_bytes": attn + append, "attn_bytes": attn,
                # the append kernel wkv_append(_fp8) picks for T = 16,384 tokens: the bulk paths
                # from 256 (bf16) / 64 (fp8) tokens on
                "kernel": ("prefill_gqa_kernel<128,true> (+ append_fp8_bulk_kernel)" if fp8 else
                           "prefill_gqa_kernel<128,false> (+ append_bf16_bulk_kernel)"),
                "dtype": "bf16" + (" (fp8-e4m3 KV)" if fp8 else ""),
                "flops_per_layer": flops, "cache_bytes": caches[0].nbytes, "bound": "mfma",
                "desc": f"Qwen3-4B prompt step: {args.layers} layers x (append + causal prefill attention), "
                        f"{B} prompts x {n_new} tokens, 32 q / 8 kv heads, d=128, {kv_dtype} KV, block 16"}
    elif name in ("sampler", "sampler-default"):
        # the step after decode: one token per row from bf16 logits over Qwen's vocabulary with
        # processed logprobs and the sampling mask; "sampler": temperature 0.7, top_k 50, top_p 0.9;
        # "sampler-default": the RL sampling defaults (temperature 1, top_p 1, top_k and min_p off,
        # configs/config.py:854-859), which draw from the whole row
        from wavelet_amd import sample
        B, V = 256, 151936
        # per-row parameter tensors and outputs made once, as a serving loop keeps them
        per_row = ({"temperature": (0.7, torch.float32), "top_k": (50, torch.int32), "top_p": (0.9, torch.float32)}
                   if name == "sampler" else {"temperature": (1.0, torch.float32)})
        params = {k: torch.full((B,), v, dtype=dt, device=dev) for k, (v, dt) in per_row.items()}
        outs = (torch.empty(B, dtype=torch.int64, device=dev), torch.empty(B, dtype=torch.float32, device=dev),
                torch.empty((B, (V + 31) // 32), dtype=torch.int32, device=dev),
                torch.empty(B, dtype=torch.int32, device=dev))
        gen = torch.Generator(device=dev)
        gen.manual_seed(1234)
        # four logits buffers in turn (311 MB, beyond the 256 MB last-level cache): no call re-reads a cached row
        logits = [(torch.randn((B, V), generator=gen, device=dev) * 4).to(torch.bfloat16) for _ in range(4)]
        seeds = torch.arange(B, dtype=torch.int64, device=dev)

        class _Step:
            grouped = False

            def __init__(self):
                self.n = 0

            def step_layer(self, layer):
                self.n += 1
                sample(logits[self.n % 4], seeds=seeds, step=self.n, return_mask=True, out=outs, **params)

            def run(self):
                self.step_layer(0)

        args.layers = 1
        w = synth.make_decode_workload(name, batch=B, num_kv_heads=1, num_q_heads=1, head_dim=64, block_size=16,
                                       context_lens=np.ones(B))
        words = (V + 31) // 32
        nbytes = B * V * 2 + B * (8 + 4 + 4) + B * words * 4
        return {"name": name, "step": _Step(), "w": w, "layer_bytes": nbytes, "attn_bytes": nbytes, "split": False,
                "kernel": "sample_kernel<bf16>", "dtype": "bf16 logits, fp32 math", "flops_per_layer": 0,
                "metric": "sampler GB/s of logits & us/step, 256 x 151936",
                "cache_bytes": 4 * B * V * 2,
                "desc": f"token sampler: {B} rows x {V} bf16 logits, "
                        + ("T=0.7, top_k=50, top_p=0.9" if name == "sampler" else "T=1, top_p=1, no top_k / min_p")
                        + ", processed logprobs + sampling mask"}
    else:
        raise SystemExit(f"unknown workload {name}")
    L = w.context_lens.astype(np.int64)
    B, HQ, HKV, D, BS = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size
    used = np.unique(np.concatenate([w.block_tables[i, :(int(L[i]) + BS - 1) // BS] for i in range(B)]))
    kv_unique = len(used) * BS * 2 * HKV * D * kv_bytes  # physical blocks read (shared prompts counted once)
    if w.group_size == 1:
        kv_unique = int(L.sum()) * 2 * HKV * D * kv_bytes
    scales = len(used) * 2 * HKV * 4 if kv_bytes == 1 else 0
    attn = kv_unique + scales + B * HQ * D * 2 * 2 + int(((L + BS - 1) // BS).sum()) * 4 + B * 4
    append = B * 2 * HKV * D * (2 + kv_bytes) + B * 8
    f8 = "true" if kv_bytes == 1 else "false"
    return {"name": name, "step": step, "w": w, "layer_bytes": attn + append, "attn_bytes": attn,
            "kernel": f"decode_gqa_kernel<{D},{f8},true,W,RP>",
            "dtype": "fp8_e4m3 KV, bf16 q/o" if kv_bytes == 1 else "bf16", "desc": desc, "kv_dtype": kv_dtype,
            "flops_per_layer": 4 * int(L.sum()) * HQ * D, "cache_bytes": cache_bytes,
            "logical_kv_bytes": int(L.sum()) * 2 * HKV * D * kv_bytes,
            "stream": (w.group_size == 1) if stream is None else stream}


def phase_clocks(args) -> int:
    """Per-phase shader-clock cycles of the MLA decode kernel, from the profiling
    build of the library (libwkv_phase.so, compiled with WKV_PHASE_CLOCKS): one
    warm pass over the layers, then one layer's launch, then the medians over
    its workgroups of each phase's cycles per step."""
    import ctypes

    import wavelet_amd._lib as L
    from wavelet_amd.build import PHASE_LIB

    if args.workload != "deepseek-v3-mla":
        print("--phase-clocks applies to the deepseek-v3-mla workload", file=sys.stderr)
        return 2
    if not PHASE_LIB.exists():
        print(f"{PHASE_LIB} is missing: python -m wavelet_amd.build --phase-clocks", file=sys.stderr)
        return 2
    L.LIB_PATH = PHASE_LIB
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    wl = workload(args, torch, dev)
    step = wl["step"]
    for _ in range(3):
        for layer in range(args.layers):
            step.attend(layer)
    torch.cuda.synchronize()
    step.attend(0)
    torch.cuda.synchronize()
    lib = L.load()
    lib.wkv_mla_phase_clocks.restype = ctypes.c_int
    lib.wkv_mla_phase_clocks.argtypes = [ctypes.c_void_p, ctypes.c_int]
    n = 1024 * 16
    buf = np.zeros(n, np.uint64)
    if lib.wkv_mla_phase_clocks(buf.ctypes.data, n) != 0:
        print("reading the phase clocks failed", file=sys.stderr)
        return 1
    r = buf.reshape(-1, 16).astype(np.float64)
    r = r[r[:, 2] > 0]
    steps = r[:, 2]
    med = lambda i: round(float(np.median(r[:, i] / steps)), 1)
    res = {
        "metric": "MLA decode phase cycles (s_memtime, median workgroup)", "workload": wl["desc"],
        "workgroups": int(len(r)), "steps": int(np.median(steps)),
        "cycles_per_workgroup": round(float(np.median(r[:, 0])), 0),
        "wall_us_per_workgroup": round(float(np.median(r[:, 1])) / 100.0, 2),
        "shader_clock_ghz": round(float(np.median(r[:, 0] / (r[:, 1] * 10.0))), 3),
        "launch_wall_us": round(float(r[:, 13].max() - r[:, 12].min()) / 100.0, 2),
        "per_step": {
            "copy": {"barrier": med(3), "issue": med(4), "wait": med(5)},
            "pv": {"barrier": med(8), "operand_reads": med(9), "mfma": med(10)},
            "qk": {"barrier": med(11), "mfma": med(14), "softmax": med(15)},
        },
        "prologue": {"copy": round(float(np.median(r[:, 7])), 0), "pv": round(float(np.median(r[:, 6])), 0)},
    }
    print(json.dumps(res))
    return 0


def main() -> int:
    args = parse()
    if args.calibrate_copy:
        return calibrate_copy()
    if args.phase_clocks:
        return phase_clocks(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); run it with --gpus 1", file=sys.stderr)
        return 2
    if args.kv_dtype is not None and args.workload in NO_KV_DTYPE:
        print(f"--kv-dtype does not apply to the {args.workload} workload", file=sys.stderr)
        return 2
    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    wl = workload(args, torch, dev)
    step, w = wl["step"], wl["w"]
    torch.cuda.synchronize()
    print(f"# setup done: {wl['name']}, {args.layers} layers x {wl['cache_bytes'] / 2**30:.2f} GiB cache",
          file=sys.stderr, flush=True)

    def timed(run) -> tuple[float, float]:
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            run()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps, (time.perf_counter() - t0) / args.steps * 1e3

    ms_per_step, wall_ms = timed(step.run)
    print(f"# timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step (wall {wall_ms:.2f} ms/step)",
          file=sys.stderr, flush=True)
    graph_rec = None
    if args.graph:
        from wavelet_amd.plan import DecodeStep, GraphDecodeStep

        plain = step.step if hasattr(step, "shared_blocks") else step
        if not isinstance(plain, DecodeStep) or plain.grouped:
            print("--graph applies to the plain GQA decode workloads", file=sys.stderr)
            return 2
        graph = GraphDecodeStep(plain, shared_blocks=getattr(step, "shared_blocks", None))
        eager_ms = ms_per_step
        ms_per_step, wall_ms = timed(graph.replay)
        graph_rec = {"us_per_step_replayed": round(ms_per_step * 1e3, 1), "us_per_step_eager": round(eager_ms * 1e3, 1),
                     "launch": "one HIP graph per step: decode order + every layer's allocation-free fused "
                               "append + attention (wkv_append_paged_decode_gqa_noalloc)"}
        print(f"# graph replays: {ms_per_step * 1e3:.1f} us/step (eager {eager_ms * 1e3:.1f})", file=sys.stderr,
              flush=True)

    # Per-launch timing of one layer's step (fused append + attention for GQA),
    # layer caches rotated so no layer is re-read from cache.
    def per_launch(fn, reps):
        # one event pair around each pass of back-to-back launches over all layers:
        # the mean device time per layer call, without a gap per launch
        # (at least 8 launches a pass: one pass of a one-launch step would time the host's launch gap)
        n = max(args.layers, 8)
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in pairs:
            a.record()
            for i in range(n):
                fn(i % args.layers)
            b.record()
        torch.cuda.synchronize()
        return float(np.mean([a.elapsed_time(b) for a, b in pairs])) * 1e3 / n

    kernel_us = per_launch(step.step_layer, args.kernel_reps)
    split = wl.get("split", True)  # the step has separate append and attention calls
    attend_us = per_launch(step.attend, 1) if split else None
    append_us = per_launch(step.append, 1) if split else None
    ceiling = hbm_read_ceiling_gbs(torch, dev)

    step_bytes = wl["layer_bytes"] * args.layers
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = wl["layer_bytes"] / (kernel_us * 1e-6) / 1e9
    headline = (wl["name"] == "qwen3-4b" and wl.get("kv_dtype") == "bf16" and w.batch == 64
                and int(w.context_lens.max()) == 4096 and args.layers == 36)
    B = w.batch
    if wl.get("bound") == "mfma":  # compute-bound workload: TFLOP/s against the dense bf16 MFMA peak
        tflops_step = wl["flops_per_layer"] * args.layers / (ms_per_step * 1e-3) / 1e12
        tflops_launch = wl["flops_per_layer"] / (kernel_us * 1e-6) / 1e12
        rec = {
            "metric": f"prefill attention TFLOP/s & us/step, {wl['name']}",
            "value": round(tflops_step, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "us_per_step": round(ms_per_step * 1e3, 1),
            "mfma_frac": round(tflops_step / MFMA_PEAK_BF16_TFLOPS, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": wl["dtype"],
            "data": "synthetic (random q/K/V, seeded), resident in HBM",
            "config": {"workload": wl["desc"], "layers": args.layers, "batch": B,
                       "q_heads": w.num_q_heads, "kv_heads": w.num_kv_heads, "head_dim": w.head_dim,
                       "block_size": w.block_size, "flops_per_step": wl["flops_per_layer"] * args.layers},
            "roofline": {"bound": "mfma", "kernel": wl["kernel"], "achieved": round(tflops_launch, 1),
                         "peak": MFMA_PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops_launch / MFMA_PEAK_BF16_TFLOPS, 4), "traffic": None,
                         "mean_launch_us": round(kernel_us, 2), "hbm_gbs": round(achieved, 1)},
            "unfused_us": {"append": round(append_us, 2), "attention": round(attend_us, 2)},
        }
        print(json.dumps(rec), flush=True)
        return 0
    kernel_name = wl["kernel"]
    if ",W,RP>" in kernel_name:  # the GQA decode: the library's waves per workgroup for this geometry
        from wavelet_amd import decode_plan

        _, waves, _ = decode_plan(w.batch, w.num_kv_heads, int(w.context_lens.max()), w.block_size, args.partition)
        # read policy: 0 cached (shared blocks), 1 streamed, 2 the group split (prompt cached, own tokens streamed)
        rp = 2 if getattr(step, "grouped", False) else (1 if wl["stream"] else 0)
        kernel_name = kernel_name.replace(",W,RP>", f",{waves},{rp}>")
    rec = {
        "metric": "decode-attn+KV-append GB/s (% of HBM peak) & us/step, Qwen3-4B B=64 4k ctx" if headline
        else wl.get("metric", f"decode-attn+KV-append GB/s & us/step, {wl['name']}"),
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
        "dtype": wl["dtype"],
        "data": "synthetic (random K/V/q, seeded), resident in HBM",
        "config": {
            "workload": wl["desc"],
            "layers": args.layers, "batch": B, "context": int(w.context_lens.max()) if headline else
            [int(w.context_lens.min()), int(w.context_lens.max())],
            "q_heads": w.num_q_heads, "kv_heads": w.num_kv_heads, "head_dim": w.head_dim,
            "block_size": w.block_size, "partition_size": args.partition or "auto", "bytes_per_step": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": wl["layer_bytes"],
            "mean_launch_us": round(kernel_us, 2),
            "tflops": round(wl["flops_per_layer"] / (kernel_us * 1e-6) / 1e12, 2),
            "frac_of_read_ceiling": round(achieved / ceiling["gbs"], 4) if ceiling["gbs"] else None,
        },
        "hbm_read_ceiling_gbs": ceiling["gbs"],
        "hbm_read_ceiling": {"kernel": "hbm_read_probe_kernel (16-byte loads, 8 in flight per lane)",
                             "bytes": ceiling["bytes"], "workgroups": ceiling["workgroups"]},
    }
    if args.via_pool:
        rec["config"]["via_pool"] = True
    if graph_rec is not None:
        rec["graph"] = graph_rec
    traffic, source = measured_traffic(wl["name"], wl.get("kv_dtype", ""), kernel_name)
    if traffic is not None and not args.via_pool and args.layers == ({"qwen3-4b": 36, "qwen3-4b-var": 36, "qwen2.5-0.5b": 24,
                                                "deepseek-v3-mla": 8}
                                               .get(wl["name"], -1)) and args.partition == 0:
        rec["roofline"]["traffic"] = traffic
        rec["roofline"]["traffic_source"] = source
    if split:
        rec["unfused_us"] = {"append": round(append_us, 2), "attention": round(attend_us, 2)}
    if "logical_kv_bytes" in wl and wl["w"].group_size > 1:
        rec["config"]["logical_kv_bytes_per_layer"] = wl["logical_kv_bytes"]
    if headline and not args.no_cpu_baseline and not args.via_pool:
        rec["cpu_baseline"] = cpu_baseline(args, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size, w.scale,
                                           wl["layer_bytes"])
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
