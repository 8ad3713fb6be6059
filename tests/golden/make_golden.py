"""Writes the golden fixtures of the KV path (run from the repository root).

    python tests/golden/make_golden.py

Every fixture is inputs plus expected outputs computed by the oracle
(``oracle/``), which is itself pinned against library routines and the
reference's own known answer in tests/test_oracle.py. The reference cannot
produce these vectors: its KV arithmetic lives in vLLM 0.28.0, which is not
vendored in the reference tree and is not installed here. The fixtures freeze
the oracle's outputs so that a later change to the oracle or to the synthetic
generator is caught, and they give the GPU tests small ready-made cases.

Inputs come from the repo-local seeded generator (wavelet_amd.synth), whose
bytes checksums.json pins; large expected outputs are stored as SHA-256
digests, small ones as arrays. Files (numpy .npz without pickles, JSON):
  outputs.json        append+gather on 4 sequences of the 1-layer workload
                      (8 KV heads x 128, block 16): digests of the inputs, of
                      the cache after a prefill and a decode append, and of the
                      gathered context; digest of the GQA decode inputs
  fp8_block.npz       one (block, head) through an fp8 prefill run and three
                      decode appends with scale growth: inputs, codes, scales
  gqa_decode.npz      float64 oracle output of a 3-sequence GQA decode
                      (32 q / 8 kv heads, d=128)
  ignore_slot.npz     the reference's ignore-slot known answer (NaN in every
                      never-read slot, output sigmoid(0.625)*[2,-1])
  checksums.json      SHA-256 of the synthetic inputs of every workload
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import paged  # noqa: E402
from wavelet_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def slots_for(w, lo, hi):
    out = []
    for i in range(w.batch):
        pos = np.arange(int(lo[i]), int(hi[i]))
        out.append(w.block_tables[i][pos // w.block_size].astype(np.int64) * w.block_size + pos % w.block_size)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def append_gather_case():
    """Inputs of the append+gather fixture (regenerated from the seeded generator)."""
    w = synth.append_gather_workload(seqs=4, max_len=100, num_blocks=64)
    h, d = w.num_kv_heads, w.head_dim
    ctx = w.context_lens.astype(np.int64)
    pslots = slots_for(w, np.zeros(w.batch, np.int64), ctx - 1)
    kp = synth.normal_bf16(synth.stream_key("golden-ag", "pk"), (len(pslots), h, d))
    vp = synth.normal_bf16(synth.stream_key("golden-ag", "pv"), (len(pslots), h, d))
    nslots = w.new_token_slots()
    kn = synth.normal_bf16(synth.stream_key("golden-ag", "nk"), (w.batch, h, d))
    vn = synth.normal_bf16(synth.stream_key("golden-ag", "nv"), (w.batch, h, d))
    return w, pslots, kp, vp, nslots, kn, vn


def append_gather() -> dict:
    w, pslots, kp, vp, nslots, kn, vn = append_gather_case()
    kc, vc = paged.empty_cache(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, fill=0xFFFF)
    paged.append_bf16(kc, vc, kp, vp, pslots)
    paged.append_bf16(kc, vc, kn, vn, nslots)
    gk, gv = paged.gather(kc, vc, w.block_tables, w.context_lens)
    return {"inputs": synth.sha256_of(w.block_tables, w.context_lens, pslots, kp, vp, nslots, kn, vn),
            "k_cache": synth.sha256_of(kc), "v_cache": synth.sha256_of(vc),
            "gathered_k": synth.sha256_of(gk), "gathered_v": synth.sha256_of(gv)}


def fp8_block():
    nb, bs, h, d = 4, 16, 1, 128
    kc, vc = paged.empty_cache(nb, bs, h, d, dtype=np.uint8)
    ks = np.zeros((nb, h), np.float32)
    vs = np.zeros((nb, h), np.float32)
    calls = [(np.arange(2 * bs, 2 * bs + 6, dtype=np.int64), 1.0), (np.array([2 * bs + 6], np.int64), 30.0),
             (np.array([2 * bs + 7], np.int64), 0.01), (np.array([2 * bs + 8], np.int64), 700.0)]
    inputs = {}
    for i, (sl, mag) in enumerate(calls):
        k = synth.normal_bf16(synth.stream_key("golden-fp8", i, "k"), (len(sl), h, d), std=mag)
        v = synth.normal_bf16(synth.stream_key("golden-fp8", i, "v"), (len(sl), h, d), std=mag / 2)
        paged.append_fp8(kc, vc, ks, vs, k, v, sl)
        inputs[f"slots{i}"], inputs[f"k{i}"], inputs[f"v{i}"] = sl, k, v
    np.savez_compressed(OUT / "fp8_block.npz", k_cache=kc, v_cache=vc, k_scale=ks, v_scale=vs, **inputs)


def gqa_decode_case():
    w = synth.make_decode_workload("golden-gqa", batch=3, num_kv_heads=8, num_q_heads=32, head_dim=128,
                                   block_size=16, context_lens=np.array([1, 37, 300]))
    shape = (w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim)
    k = synth.normal_bf16(synth.stream_key("golden-gqa", "k"), shape)
    v = synth.normal_bf16(synth.stream_key("golden-gqa", "v"), shape)
    q = synth.normal_bf16(synth.stream_key("golden-gqa", "q"), (w.batch, 32, 128))
    return w, k, v, q


def gqa_decode() -> str:
    w, k, v, q = gqa_decode_case()
    out = paged.decode_gqa(paged.bf16_to_f32(q), paged.bf16_to_f32(k), paged.bf16_to_f32(v), w.block_tables,
                           w.context_lens, w.scale)
    np.savez_compressed(OUT / "gqa_decode.npz", out=out)
    return synth.sha256_of(w.block_tables, w.context_lens, k, v, q)


def ignore_slot():
    nb, bs, h, d = 2, 16, 1, 64
    kc = np.full((nb, bs, h, d), np.nan, np.float32)
    vc = np.full((nb, bs, h, d), np.nan, np.float32)
    kc[1, 0], vc[1, 0] = 0.0, 0.0
    kc[1, 1], vc[1, 1] = 0.0, 0.0
    kc[1, 1, 0, :2] = [2.0, -1.0]
    vc[1, 1, 0, :2] = [2.0, -1.0]
    q = np.zeros((1, 1, d), np.float32)
    q[0, 0, :2] = [0.5, -0.25]
    expected = np.zeros((1, 1, d))
    expected[0, 0, :2] = (1.0 / (1.0 + math.exp(-0.625))) * np.array([2.0, -1.0])
    np.savez_compressed(OUT / "ignore_slot.npz", k_logical=kc, v_logical=vc, q=q, block_tables=np.array([[1]], np.int32),
                        context_lens=np.array([2], np.int32), scale=np.float64(0.5), expected=expected)


def checksums() -> dict:
    """SHA-256 of each workload's generated inputs (tables, lengths, leading tensors)."""
    out = {}
    for name, w in [("append_gather", synth.append_gather_workload()),
                    ("qwen2.5-0.5b", synth.qwen25_05b_workload()),
                    ("qwen3-4b", synth.qwen3_4b_workload()),
                    ("qwen3-4b-var", synth.qwen3_4b_workload(context=None)),
                    ("qwen2.5-7b-groups", synth.qwen25_7b_group_workload()),
                    ("deepseek-v3-mla", synth.deepseek_v3_mla_workload())]:
        q = synth.normal_bf16(synth.stream_key(w.name, "checksum-q"), (min(w.batch, 4), w.num_q_heads, w.head_dim))
        out[name] = {
            "tables": synth.sha256_of(w.block_tables, w.context_lens),
            "q": synth.sha256_of(q),
            "num_blocks": int(w.num_blocks),
            "tokens": int(w.context_lens.astype(np.int64).sum()),
        }
    return out


def main() -> None:
    fp8_block()
    ignore_slot()
    digests = {"append_gather": append_gather(), "gqa_decode_inputs": gqa_decode()}
    (OUT / "outputs.json").write_text(json.dumps(digests, indent=2, sort_keys=True) + "\n")
    (OUT / "checksums.json").write_text(json.dumps(checksums(), indent=2, sort_keys=True) + "\n")
    for f in sorted(OUT.glob("*.npz")) + sorted(OUT.glob("*.json")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
