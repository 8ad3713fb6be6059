"""The decode's per-step read policy and the pool sized from the real device memory.

A decode step streams K/V past the caches (non-temporal loads) when no block of the
step is held by two sequences, and keeps K/V cached otherwise; the choice is made
per step from the block manager's reference counts (``KVPool.decode_shares_blocks``)
and passed per call. Both policies compute the same thing: outputs and caches are
bit-identical between them, and match the oracle.
"""

import math

import numpy as np
import pytest
import torch

from kvcase import bits_of, check_attention
from oracle import fp8, paged
from wavelet_amd import KVPool, paged_decode_gqa
from wavelet_amd.plan import DecodeStep

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _pool_with_sequences(cuda, kv_dtype: str, seed: int):
    """A 2-layer pool: three independent sequences and a group of four forked from a
    prompt that ends inside a block, their prompts written to every layer."""
    H, D, BS = 4, 128, 16
    pool = KVPool(2, 256, BS, H, D, kv_dtype, device=cuda)
    m = pool.blocks
    gen = torch.Generator(device=cuda)
    gen.manual_seed(seed)
    for sid, n in (("a", 300), ("b", 17), ("c", 1025), ("g0", 700)):
        m.allocate(sid, np.arange(n) + 10_000 * len(sid) + n, cache_salt=sid)
        pos = np.arange(n)
        slots = torch.from_numpy(np.asarray(m.blocks_of(sid), np.int64)[pos // BS] * BS + pos % BS).to(cuda)
        for c in pool.layers:
            k = torch.randn((n, H, D), generator=gen, device=cuda).to(BF16)
            v = torch.randn((n, H, D), generator=gen, device=cuda).to(BF16)
            c.append(k, v, slots)
    for j in range(1, 4):
        m.fork("g0", f"g{j}")
    return pool


def test_decode_shares_blocks_follows_the_step(cuda):
    pool = _pool_with_sequences(cuda, "bf16", 1)
    assert not pool.decode_shares_blocks(["a", "b", "c"])
    assert pool.decode_shares_blocks(["a", "g1"])  # g1 holds the group's prompt blocks
    for j in range(1, 4):
        pool.blocks.free(f"g{j}")
    assert not pool.decode_shares_blocks(["a", "b", "c", "g0"])
    assert pool.layers[0].shared_blocks  # a pool's default: blocks may be shared
    assert pool.layers[0].descriptor(False).flags == 0 and pool.layers[0].descriptor(True).flags == 1


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
def test_step_read_policy_gives_identical_results(cuda, kv_dtype):
    """Two identical pools, one step each through DecodeStep.run(shared_blocks=...) with the
    policy the pool computes and with the other one: caches and outputs bit-identical, and
    within the attention bar of the oracle. The batch holds the forked group, so the
    computed policy is the cached one; a second batch of independent sequences streams."""
    pools = [_pool_with_sequences(cuda, kv_dtype, 2) for _ in range(2)]  # same seed: identical pools
    fp8_cache = kv_dtype == "fp8_e4m3"
    for ids, expect_shared in ((["a", "g0", "b", "g1", "g2", "c", "g3"], True), (["a", "b", "c"], False)):
        outs = []
        for n, pool in enumerate(pools):
            slots = pool.append_slots(ids)
            bt, lens = pool.blocks.tables(ids)
            B = len(ids)
            gen = torch.Generator(device=cuda)
            gen.manual_seed(len(ids))
            q = [torch.randn((B, 16, 128), generator=gen, device=cuda).to(BF16) for _ in range(2)]
            k = [torch.randn((B, 4, 128), generator=gen, device=cuda).to(BF16) for _ in range(2)]
            v = [torch.randn((B, 4, 128), generator=gen, device=cuda).to(BF16) for _ in range(2)]
            o = [torch.empty((B, 16, 128), dtype=BF16, device=cuda) for _ in range(2)]
            step = DecodeStep(pool.layers, q, k, v, o, torch.from_numpy(bt).to(cuda),
                              torch.from_numpy(lens).to(cuda), slots, 1 / math.sqrt(128), int(lens.max()),
                              partition_size=64)  # several partitions and the merge kernel
            shared = pool.decode_shares_blocks(ids)
            assert shared == expect_shared
            step.run(shared_blocks=shared if n == 0 else not shared)
            torch.cuda.synchronize()
            outs.append((o, q, bt, lens))
        for layer in range(2):
            a, b = pools[0].layers[layer], pools[1].layers[layer]
            assert torch.equal(a.k.view(torch.uint8), b.k.view(torch.uint8)), f"K differs, layer {layer}"
            assert torch.equal(a.v.view(torch.uint8), b.v.view(torch.uint8)), f"V differs, layer {layer}"
            if fp8_cache:
                assert torch.equal(a.k_scale, b.k_scale) and torch.equal(a.v_scale, b.v_scale)
            o0, o1 = outs[0][0][layer], outs[1][0][layer]
            assert torch.equal(o0.view(torch.int16), o1.view(torch.int16)), f"output differs, layer {layer}"
            # and the oracle, on the cache after the step
            kb, vb = bits_of(a.k), bits_of(a.v)
            if fp8_cache:
                nb = kb.shape[0]
                kf = fp8.dequantize(paged.k_logical(kb).reshape(nb, 16, 4, 128),
                                    a.k_scale.cpu().numpy()[:, None, :, None])
                vf = fp8.dequantize(paged.v_logical(vb), a.v_scale.cpu().numpy()[:, None, :, None])
            else:
                kl, vl = paged.logical_kv(kb, vb)
                kf, vf = paged.bf16_to_f32(kl), paged.bf16_to_f32(vl)
            _, q, bt, lens = outs[0]
            ref = paged.decode_gqa(paged.bf16_to_f32(bits_of(q[layer])), kf, vf, bt, lens, 1 / math.sqrt(128))
            check_attention(paged.bf16_to_f32(bits_of(o0)), ref, f"policy {kv_dtype} layer {layer}")


def test_pool_sized_from_device_memory(cuda):
    """KVPool.from_engine_config with the real torch.cuda.mem_get_info: the pool holds no more
    than gpu_memory_utilization x total - reserve, the block count is the engine's formula,
    metrics_text() reports it, and a decode runs through the pool."""
    free, total = torch.cuda.mem_get_info(cuda)
    util, reserve, non_kv = 0.05, 512 << 20, 256 << 20
    pool = KVPool.from_engine_config(num_layers=4, num_kv_heads=8, head_dim=128, block_size=16,
                                     gpu_memory_utilization=util, max_model_len=8192, non_kv_bytes=non_kv,
                                     reserve_bytes=reserve, device=cuda)
    per_block = 4 * 2 * 16 * 8 * 128 * 2
    assert pool.num_blocks == (int(util * total) - non_kv - reserve) // per_block
    assert pool.nbytes <= util * total - reserve - non_kv
    assert f'num_gpu_blocks="{pool.num_blocks}"' in pool.metrics_text()
    used = torch.cuda.memory_allocated(cuda)
    assert used >= pool.nbytes
    m = pool.blocks
    m.allocate("s", np.arange(100))
    bt, lens = m.tables(["s"])
    assert bt.shape[1] == 8192 // 16  # the table width max_model_len implies
    pos = np.arange(100)
    slots = torch.from_numpy(np.asarray(m.blocks_of("s"), np.int64)[pos // 16] * 16 + pos % 16).to(cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(4)
    k = torch.randn((100, 8, 128), generator=g, device=cuda).to(BF16)
    v = torch.randn((100, 8, 128), generator=g, device=cuda).to(BF16)
    pool.layers[3].append(k, v, slots)
    q = torch.randn((1, 32, 128), generator=g, device=cuda).to(BF16)
    out = paged_decode_gqa(q, pool.layers[3], torch.from_numpy(bt).to(cuda), torch.from_numpy(lens).to(cuda),
                           1 / math.sqrt(128), shared_blocks=pool.decode_shares_blocks(["s"]))
    qf = q.float()[0].view(8, 4, 128)
    s = torch.einsum("hgd,thd->hgt", qf, k.float()) / math.sqrt(128)
    ref = torch.einsum("hgt,thd->hgd", torch.softmax(s, -1), v.float()).reshape(32, 128)
    torch.testing.assert_close(out.float()[0], ref, atol=2e-2, rtol=1e-2)
