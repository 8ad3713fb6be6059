"""Dispatch order of the GQA decode.

The device order equals numpy's stable descending argsort of the lengths
(ties by index, negative lengths included); a decode dispatched in any order
-- that one, a random permutation, the batch order -- gives bit-identical
outputs and, with the fused append, a bit-identical cache, because every
(sequence, KV head) is computed by the same waves whatever the order.
"""

import numpy as np
import pytest
import torch

from kvcase import slots_for, to_dev_bits
from wavelet_amd import PagedKVCache, decode_order, paged_decode_gqa, synth
from wavelet_amd.plan import DecodeStep

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


@pytest.mark.parametrize("batch", [1, 7, 64, 256, 300, 3000])
def test_decode_order_is_stable_descending_argsort(cuda, batch):
    rng = np.random.default_rng(batch)
    lens = rng.integers(0, 50, batch).astype(np.int32)  # many ties
    k = max(batch // 5, 1)
    lens[:k] = rng.integers(-3, 9000, k)
    got = decode_order(torch.from_numpy(lens).to(cuda)).cpu().numpy()
    np.testing.assert_array_equal(got, np.argsort(-lens.astype(np.int64), kind="stable"))


def _caches(cuda, w, kv_dtype, n, last=False):
    """n caches with identical contents: every context position written, but
    the last (which a fused append writes) unless ``last``."""
    caches = [PagedKVCache(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, kv_dtype=kv_dtype, device=cuda)
              for _ in range(n)]
    ctx = w.context_lens.astype(np.int64)
    slots = slots_for(w, np.zeros(w.batch, np.int64), ctx if last else np.maximum(ctx - 1, 0))
    k = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "k"), (len(slots), w.num_kv_heads, w.head_dim)),
                    BF16, cuda)
    v = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "v"), (len(slots), w.num_kv_heads, w.head_dim)),
                    BF16, cuda)
    for c in caches:
        c.append(k, v, torch.from_numpy(slots).to(cuda))
    return caches


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
@pytest.mark.parametrize("fused", [False, True])
def test_decode_in_any_order_is_bit_identical(cuda, kv_dtype, fused):
    lens = np.array([1, 5000, 17, 300, 2049, 64, 1025, 4097, 33, 16])
    hq, hkv, d, bs = 32, 8, 128, 16
    w = synth.make_decode_workload(f"order{kv_dtype}", batch=len(lens), num_kv_heads=hkv, num_q_heads=hq,
                                   head_dim=d, block_size=bs, context_lens=lens)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    q = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, hq, d)), BF16, cuda)
    kn = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "nk"), (w.batch, hkv, d)), BF16, cuda)
    vn = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "nv"), (w.batch, hkv, d)), BF16, cuda)
    nslots = torch.from_numpy(w.new_token_slots()).to(cuda)
    desc = decode_order(sl)
    rand = torch.from_numpy(np.random.default_rng(5).permutation(w.batch).astype(np.int32)).to(cuda)
    for p in (0, 4 * bs):
        caches = _caches(cuda, w, kv_dtype, 3, last=not fused)
        outs = []
        for cache, order in zip(caches, (None, desc, rand)):
            extra = dict(new_key=kn, new_value=vn, slot_mapping=nslots) if fused else {}
            outs.append(paged_decode_gqa(q, cache, bt, sl, w.scale, partition_size=p, seq_order=order, **extra))
        torch.cuda.synchronize()
        for i in (1, 2):
            assert torch.equal(outs[i].view(torch.int16), outs[0].view(torch.int16)), f"order {i}, P={p}: output"
            assert torch.equal(caches[i].k.view(torch.uint8), caches[0].k.view(torch.uint8)), f"order {i}: K"
            assert torch.equal(caches[i].v.view(torch.uint8), caches[0].v.view(torch.uint8)), f"order {i}: V"
            if kv_dtype == "fp8_e4m3":
                assert torch.equal(caches[i].k_scale, caches[0].k_scale)
                assert torch.equal(caches[i].v_scale, caches[0].v_scale)


def test_decode_step_orders_by_length_bit_identically(cuda):
    """DecodeStep over 2 layers with its per-step order equals the batch-order step, twice in a row."""
    lens = np.array([3000, 12, 700, 4096, 1, 2500, 90, 1600])
    hq, hkv, d = 28, 4, 128
    w = synth.make_decode_workload("orderstep", batch=len(lens), num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=16, context_lens=lens)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    nslots = torch.from_numpy(w.new_token_slots()).to(cuda)
    layers = 2
    q = [to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "q", str(i)), (w.batch, hq, d)), BF16, cuda)
         for i in range(layers)]
    kn = [to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "k", str(i)), (w.batch, hkv, d)), BF16, cuda)
          for i in range(layers)]
    vn = [to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "v", str(i)), (w.batch, hkv, d)), BF16, cuda)
          for i in range(layers)]
    results = []
    for ordered in (False, True):
        caches = [_caches(cuda, w, "bf16", 1)[0] for _ in range(layers)]
        out = [torch.empty((w.batch, hq, d), dtype=BF16, device=cuda) for _ in range(layers)]
        step = DecodeStep(caches, q, kn, vn, out, bt, sl, nslots, w.scale, int(lens.max()),
                          order_by_length=ordered)
        for _ in range(2):
            step.run()
        torch.cuda.synchronize()
        if ordered:
            np.testing.assert_array_equal(step.order.cpu().numpy(), np.argsort(-lens, kind="stable"))
        results.append(([o.clone() for o in out], [c.k.clone() for c in caches], [c.v.clone() for c in caches]))
    for a, b in zip(results[0], results[1]):
        for x, y in zip(a, b):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
