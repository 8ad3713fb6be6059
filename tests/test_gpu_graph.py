"""A decode step captured in a HIP graph (GraphDecodeStep) and replayed step after step.

Two identical sets of caches advance through the same four decode steps: one by the
eager DecodeStep (workspace path), one by graph replays (the allocation-free entry
point). Between steps the shared inputs are refilled in place (new q/K/V, lengths + 1,
the next slots) by ordinary eager work, with synchronisations between the replays.
After every replay the outputs and the whole caches equal the eager ones bit for bit,
and the last step is checked against the oracle.
"""

import math

import numpy as np
import pytest
import torch

from kvcase import bits_of, check_attention
from oracle import fp8, paged
from wavelet_amd import PagedKVCache, synth
from wavelet_amd.plan import DecodeStep, GraphDecodeStep

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
STEPS = 4


def _case(cuda, kv_dtype, hq, hkv, d, lens, partition, layers=3, order=None, seed=0):
    name = f"graph{kv_dtype}{hq}{hkv}{d}p{partition}"
    print(f"case {name}: B={len(lens)} L=[{min(lens)}, {max(lens)}]", flush=True)
    lens = np.asarray(lens, np.int64)
    bs = 16
    w = synth.make_decode_workload(name, batch=len(lens), num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=bs, context_lens=lens + STEPS)  # tables hold the four new tokens
    gen = torch.Generator(device=cuda)
    gen.manual_seed(seed)
    sets = []
    for _ in range(2):
        caches = [PagedKVCache(w.num_blocks, bs, hkv, d, kv_dtype=kv_dtype, device=cuda) for _ in range(layers)]
        sets.append(caches)
    # the cached contexts (positions [0, lens)), the same in both sets
    pos = [np.arange(int(L)) for L in lens]
    pslots = np.concatenate([w.block_tables[i][p // bs].astype(np.int64) * bs + p % bs for i, p in enumerate(pos)])
    pslots = torch.from_numpy(pslots).to(cuda)
    for layer in range(layers):
        k = torch.randn((len(pslots), hkv, d), generator=gen, device=cuda).to(BF16)
        v = torch.randn((len(pslots), hkv, d), generator=gen, device=cuda).to(BF16)
        for caches in sets:
            caches[layer].append(k, v, pslots)
    B = len(lens)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy((lens + 1).astype(np.int32)).to(cuda)
    slots = torch.empty(B, dtype=torch.int64, device=cuda)
    q = [torch.empty((B, hq, d), dtype=BF16, device=cuda) for _ in range(layers)]
    kn = [torch.empty((B, hkv, d), dtype=BF16, device=cuda) for _ in range(layers)]
    vn = [torch.empty((B, hkv, d), dtype=BF16, device=cuda) for _ in range(layers)]
    outs = [[torch.empty((B, hq, d), dtype=BF16, device=cuda) for _ in range(layers)] for _ in range(2)]
    max_seq = int(lens.max()) + STEPS
    scale = 1 / math.sqrt(d)
    eager = DecodeStep(sets[0], q, kn, vn, outs[0], bt, sl, slots, scale, max_seq, partition_size=partition,
                       order_by_length=order)
    graph_plan = DecodeStep(sets[1], q, kn, vn, outs[1], bt, sl, slots, scale, max_seq, partition_size=partition,
                            order_by_length=order)

    def refill(t):
        p = lens + t  # the new token's position
        slots.copy_(torch.from_numpy(w.block_tables[np.arange(B), p // bs].astype(np.int64) * bs + p % bs))
        sl.copy_(torch.from_numpy((p + 1).astype(np.int32)))
        for layer in range(layers):
            q[layer].copy_(torch.randn((B, hq, d), generator=gen, device=cuda))
            kn[layer].copy_(torch.randn((B, hkv, d), generator=gen, device=cuda))
            vn[layer].copy_(torch.randn((B, hkv, d), generator=gen, device=cuda))

    refill(0)
    graph = GraphDecodeStep(graph_plan)  # captured once, with the step-0 buffers in place
    for t in range(STEPS):
        if t:
            refill(t)
        torch.cuda.synchronize()
        eager.run()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            a, b = sets[0][layer], sets[1][layer]
            assert torch.equal(a.k.view(torch.uint8), b.k.view(torch.uint8)), f"{name} step {t}: K layer {layer}"
            assert torch.equal(a.v.view(torch.uint8), b.v.view(torch.uint8)), f"{name} step {t}: V layer {layer}"
            if kv_dtype == "fp8_e4m3":
                assert torch.equal(a.k_scale, b.k_scale) and torch.equal(a.v_scale, b.v_scale)
            assert torch.equal(outs[0][layer].view(torch.int16), outs[1][layer].view(torch.int16)), \
                f"{name} step {t}: output layer {layer}"
    # the last step against the oracle, on the cache after it
    c = sets[1][-1]
    kb, vb = bits_of(c.k), bits_of(c.v)
    if kv_dtype == "fp8_e4m3":
        nb = kb.shape[0]
        kf = fp8.dequantize(paged.k_logical(kb).reshape(nb, bs, hkv, d), c.k_scale.cpu().numpy()[:, None, :, None])
        vf = fp8.dequantize(paged.v_logical(vb), c.v_scale.cpu().numpy()[:, None, :, None])
    else:
        kl, vl = paged.logical_kv(kb, vb)
        kf, vf = paged.bf16_to_f32(kl), paged.bf16_to_f32(vl)
    ref = paged.decode_gqa(paged.bf16_to_f32(bits_of(q[-1])), kf, vf, w.block_tables, (lens + STEPS).astype(np.int32),
                           scale)
    a, r = check_attention(paged.bf16_to_f32(bits_of(outs[1][-1])), ref, name)
    print(f"{name}: err abs {a:.2e} rel {r:.2e}")


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
def test_graph_replay_equals_eager_steps(cuda, kv_dtype):
    """Qwen3-4B heads, ragged lengths, the library's partition, longest-first dispatch order."""
    _case(cuda, kv_dtype, 32, 8, 128, [1, 30, 600, 2047, 4000, 100, 1023, 3000], 0, order=True, seed=1)


def test_graph_replay_with_split_k_merge(cuda):
    """64-token partitions: several workgroups per sequence, partials merged by the second
    kernel inside the graph (its partials in the static scratch)."""
    _case(cuda, "bf16", 14, 2, 64, [5, 64, 300, 900, 2000, 17], 64, seed=2)


def test_graph_replay_qwen25_05b_geometry(cuda):
    """The Qwen2.5-0.5B layer's heads (14 / 2, d=64) at its batch of 128, lengths in [256, 2048]."""
    lens = np.random.default_rng(3).integers(256, 2048 - STEPS, 128)
    _case(cuda, "bf16", 14, 2, 64, lens.tolist(), 0, layers=2, seed=3)


def test_graph_refuses_a_geometry_beyond_the_scratch(cuda):
    B = 64
    w = synth.make_decode_workload("graphbig", batch=B, num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                                   context_lens=np.full(B, 8192))
    caches = [PagedKVCache(w.num_blocks, 16, 8, 128, device=cuda)]
    z = lambda *s: [torch.zeros(s, dtype=BF16, device=cuda)]  # noqa: E731
    step = DecodeStep(caches, z(B, 32, 128), z(B, 8, 128), z(B, 8, 128), z(B, 32, 128),
                      torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda),
                      torch.from_numpy(w.new_token_slots()).to(cuda), 0.1, 8192, partition_size=16)
    with pytest.raises(ValueError, match="scratch"):
        GraphDecodeStep(step)
