"""GPU parity of the MLA latent cache's gather and block copy (copy-on-write of a GRPO
fork whose prompt ends inside a block) -- bit-exact against the oracle -- and of the
MLA decode's attention sinks, within the attention bar of kvcase.check_attention.

The geometry is DeepSeek-V3's: 128 heads over a 512 + 64 latent row, block 64;
the gather and copy tests run at the full B=32, L=4096 workload.
"""

import math

import numpy as np
import pytest
import torch

from kvcase import assert_guards, bits_of, check_attention, guard_cache, to_dev_bits
from oracle import paged
from wavelet_amd import BlockManager, KVPool, MLALatentCache, paged_decode_mla, synth

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
R, P = 512, 64
NAN16 = np.uint16(0x7FC0)


def _random_bits_cache(cuda, num_blocks: int, bs: int, seed: int) -> MLALatentCache:
    """A latent cache holding random bit patterns (NaN and inf included): a copy must move bits."""
    gen = torch.Generator(device=cuda)
    gen.manual_seed(seed)
    c = MLALatentCache(num_blocks, bs, R, P, device=cuda)
    c.latent.view(torch.int16).copy_(torch.randint(-32768, 32768, tuple(c.latent.shape), generator=gen,
                                                   device=cuda, dtype=torch.int32).to(torch.int16))
    return c


def test_mla_gather_deepseek_v3_workload_bit_exact(cuda):
    """B=32 sequences of 4,096 tokens through a seeded permutation of the pool's blocks."""
    w = synth.deepseek_v3_mla_workload()
    print(f"case mla gather: B={w.batch} L={int(w.context_lens.max())} blocks={w.num_blocks}", flush=True)
    c = _random_bits_cache(cuda, w.num_blocks, w.block_size, 1)
    guards = guard_cache(c)
    got = c.gather(torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda))
    assert_guards(guards, "mla gather")
    assert tuple(got.shape) == (int(w.context_lens.sum()), R + P)
    np.testing.assert_array_equal(bits_of(got), paged.gather_mla(bits_of(c.latent), w.block_tables, w.context_lens))


@pytest.mark.parametrize("bs", [16, 64, 128])
def test_mla_gather_edge_lengths(cuda, bs):
    """Empty, one-token, block-boundary and ragged contexts; table entries past a context
    hold ids outside the pool (never read)."""
    lens = np.array([0, 1, bs - 1, bs, bs + 1, 3 * bs + 5, 1000, 0, 77], np.int64)
    w = synth.make_decode_workload(f"mlagather{bs}", batch=len(lens), num_kv_heads=1, num_q_heads=16, head_dim=R + P,
                                   block_size=bs, context_lens=lens)
    bt = w.block_tables.copy()
    for i, L in enumerate(lens):
        bt[i, -(-int(L) // bs):] = 1 << 30  # past the context: must never be read
    c = _random_bits_cache(cuda, w.num_blocks, bs, 2)
    got = c.gather(torch.from_numpy(bt).to(cuda), torch.from_numpy(w.context_lens).to(cuda))
    np.testing.assert_array_equal(bits_of(got), paged.gather_mla(bits_of(c.latent), bt, w.context_lens))


def test_mla_copy_blocks_bit_exact(cuda):
    """Independent copy pairs (one source feeding several destinations, pairs out of range
    skipped) over the DeepSeek-V3 workload's pool; every other block unchanged."""
    w = synth.deepseek_v3_mla_workload()
    nb = w.num_blocks
    c = _random_bits_cache(cuda, nb, w.block_size, 3)
    guards = guard_cache(c)
    lat = bits_of(c.latent)
    pairs = np.array([[5, 100], [5, 101], [7, nb - 1], [nb - 2, 0], [-1, 3], [9, nb], [11, 12]], np.int64)
    c.copy_blocks(torch.from_numpy(pairs).to(cuda))
    assert_guards(guards, "mla copy_blocks")
    paged.copy_blocks([lat], pairs)
    np.testing.assert_array_equal(bits_of(c.latent), lat)


def test_mla_grpo_fork_prompt_ending_mid_block(cuda):
    """A GRPO group of 8 on an MLA pool (2 layers): a 1,000-token prompt (its last block
    holds 40 of 64 tokens) forked to 7 siblings, three fused decode steps through
    KVPool.append_slots, which applies the block manager's copy-on-write pairs to every
    layer. Each step: the latent caches equal the oracle's (copy pairs, then the appended
    rows) bit for bit, and each member's attention over its own table matches the oracle;
    NaN fills every slot no member owns, so a member reading a sibling's private row or a
    block that was never copied shows up."""
    H, BS, NB, prompt = 128, 64, 64, 1000
    scale = 1 / math.sqrt(192.0)
    pool = KVPool(2, NB, BS, mla=True, device=cuda)
    twin = BlockManager(NB, BS)  # the same calls: the pool's pairs and slots, for the oracle
    ids = [f"g{j}" for j in range(8)]
    tokens = np.arange(prompt)
    for m in (pool.blocks, twin):
        m.allocate(ids[0], tokens, cache_salt="policy-7")
    lat = [np.full((NB, BS, R + P), NAN16, np.uint16) for _ in range(2)]
    pos = np.arange(prompt)
    pslots = np.asarray(pool.blocks.blocks_of(ids[0]), np.int64)[pos // BS] * BS + pos % BS
    for layer, c in enumerate(pool.layers):
        c.latent.copy_(to_dev_bits(lat[layer], BF16, cuda))
        kvc = synth.normal_bf16(synth.stream_key("mlagrpo", layer, "c"), (prompt, R))
        kpe = synth.normal_bf16(synth.stream_key("mlagrpo", layer, "p"), (prompt, P))
        paged.append_mla(lat[layer], kvc, kpe, pslots)
        c.append(to_dev_bits(kvc, BF16, cuda), to_dev_bits(kpe, BF16, cuda), torch.from_numpy(pslots).to(cuda))
    for m in (pool.blocks, twin):
        for g in ids[1:]:
            m.fork(ids[0], g)
    assert pool.decode_shares_blocks(ids)
    for step in range(3):
        print(f"case mla grpo step {step}", flush=True)
        slots = pool.append_slots(ids)
        tslots, cow = twin.append_slots(ids)
        np.testing.assert_array_equal(slots.cpu().numpy(), tslots)
        assert (len(cow) == 7) == (step == 0)  # only the first write into the shared partial block copies
        bt, lens = pool.blocks.tables(ids)
        for layer, c in enumerate(pool.layers):
            paged.copy_blocks([lat[layer]], cow)
            kvc = synth.normal_bf16(synth.stream_key("mlagrpo", layer, step, "nc"), (8, R))
            kpe = synth.normal_bf16(synth.stream_key("mlagrpo", layer, step, "np"), (8, P))
            q = synth.normal_bf16(synth.stream_key("mlagrpo", layer, step, "q"), (8, H, R + P))
            paged.append_mla(lat[layer], kvc, kpe, tslots)
            dq = to_dev_bits(q, BF16, cuda)
            out = paged_decode_mla(dq[:, :, :R], dq[:, :, R:], c, torch.from_numpy(bt).to(cuda),
                                   torch.from_numpy(lens).to(cuda), scale, new_kv_c=to_dev_bits(kvc, BF16, cuda),
                                   new_k_pe=to_dev_bits(kpe, BF16, cuda), slot_mapping=slots)
            assert np.array_equal(bits_of(c.latent), lat[layer]), f"latent cache, layer {layer} step {step}"
            ref = paged.decode_mla(paged.bf16_to_f32(q), paged.bf16_to_f32(lat[layer]), bt, lens, scale)
            check_attention(paged.bf16_to_f32(bits_of(out)), ref, f"mla grpo layer {layer} step {step}")
    # the prompt's full blocks stay shared; every member's block after them is its own
    bt, _ = pool.blocks.tables(ids)
    assert np.all(bt[:, :prompt // BS] == bt[0, :prompt // BS])
    assert len(set(bt[:, prompt // BS].tolist())) == 8


def _mla_sinks_case(cuda, w, sinks_np, fused: bool, partition: int, check_rows=None):
    """Decode with sinks (fused latent append or not) against the oracle; returns the output,
    the cache, the query and the fused-append arguments. Inputs come from a seeded device
    generator (N(0, 1) latent rows, NaN in every slot no context owns)."""
    H, bs = w.num_q_heads, w.block_size
    gen = torch.Generator(device=cuda)
    gen.manual_seed(sum(map(ord, w.name)))
    own = np.zeros((w.num_blocks, bs), bool)
    for i in range(w.batch):
        p = np.arange(int(w.context_lens[i]))
        own[w.block_tables[i][p // bs], p % bs] = True
    cache = MLALatentCache(w.num_blocks, bs, R, P, device=cuda)
    cache.latent.normal_(generator=gen)
    cache.latent.view(torch.int16).masked_fill_(~torch.from_numpy(own).to(cuda)[:, :, None], int(NAN16))
    dq = torch.randn((w.batch, H, R + P), generator=gen, device=cuda).to(BF16)
    kw = {}
    if fused:
        new_slots = torch.from_numpy(w.new_token_slots()).to(cuda)
        kvc = torch.randn((w.batch, R), generator=gen, device=cuda).to(BF16)
        kpe = torch.randn((w.batch, P), generator=gen, device=cuda).to(BF16)
        cache.latent.view(-1, R + P).view(torch.int16)[new_slots] = int(NAN16)  # not in the cache before the step
        kw = dict(new_kv_c=kvc, new_k_pe=kpe, slot_mapping=new_slots)
    sinks = torch.from_numpy(np.asarray(sinks_np, np.float32)).to(cuda)
    out = paged_decode_mla(dq[:, :, :R], dq[:, :, R:], cache, torch.from_numpy(w.block_tables).to(cuda),
                           torch.from_numpy(w.context_lens).to(cuda), w.scale, partition_size=partition, sinks=sinks,
                           **kw)
    torch.cuda.synchronize()
    rows = np.arange(w.batch) if check_rows is None else np.asarray(check_rows)
    # the oracle reads the cache after the step (a fused append has written the new rows)
    blocks = np.unique(np.concatenate([w.block_tables[i][:-(-int(w.context_lens[i]) // bs)] for i in rows] +
                                      [np.zeros(1, np.int32)]))
    bt = np.searchsorted(blocks, w.block_tables[rows]).astype(np.int32)
    lat = paged.bf16_to_f32(bits_of(cache.latent[torch.from_numpy(blocks).to(cuda)]))
    q = paged.bf16_to_f32(bits_of(dq[torch.from_numpy(rows).to(cuda)]))
    ref = paged.decode_mla(q, lat, bt, w.context_lens[rows], w.scale, sinks=np.asarray(sinks_np, np.float64))
    got = paged.bf16_to_f32(bits_of(out[torch.from_numpy(rows).to(cuda)]))
    a, r = check_attention(got, ref, f"mla sinks {w.name} fused={fused} P={partition}")
    print(f"mla sinks {w.name} fused={fused} P={partition}: err abs {a:.2e} rel {r:.2e}")
    return out, cache, dq, kw


def _sink_values(h: int, seed: int) -> np.ndarray:
    """Per-head sinks around the scaled scores' range, one -inf (none) and one that dominates."""
    s = np.random.default_rng(seed).normal(0.0, 2.0, h).astype(np.float32)
    s[0] = -np.inf
    s[1] = 12.0
    return s


@pytest.mark.parametrize("fused", [False, True])
def test_mla_sinks_deepseek_v3_workload(cuda, fused):
    """The bench's MLA shape (B=32, L=4096, 128 heads: four partitions merged per sequence),
    8 of the 32 sequences checked against the oracle."""
    w = synth.deepseek_v3_mla_workload()
    print(f"case mla sinks B={w.batch} fused={fused}", flush=True)
    _mla_sinks_case(cuda, w, _sink_values(128, 5), fused, 0, check_rows=np.array([0, 3, 9, 14, 18, 23, 27, 31]))


@pytest.mark.parametrize("heads,partition", [(128, 0), (128, 64), (16, 32), (64, 0), (32, 160)])
def test_mla_sinks_edge_lengths_and_partitions(cuda, heads, partition):
    """Single-partition rows (finished in the attention kernel) and merged ones (the merge
    adds the sink), an empty context (zeros) and contexts ending inside a step."""
    lens = np.array([0, 1, 17, 64, 65, 300, 1000, 2047], np.int64)
    w = synth.make_decode_workload(f"mlasink{heads}p{partition}", batch=len(lens), num_kv_heads=1, num_q_heads=heads,
                                   head_dim=R + P, block_size=64, context_lens=lens, scale=1 / math.sqrt(192.0))
    out, _, _, _ = _mla_sinks_case(cuda, w, _sink_values(heads, heads + partition), False, partition)
    assert bool((out[0] == 0).all())


@pytest.mark.parametrize("fused", [False, True])
def test_mla_minus_inf_sinks_equal_no_sinks_bit_for_bit(cuda, fused):
    lens = np.array([1, 40, 64, 129, 1500, 4096, 3, 700], np.int64)
    w = synth.make_decode_workload(f"mlasinkninf{int(fused)}", batch=len(lens), num_kv_heads=1, num_q_heads=128,
                                   head_dim=R + P, block_size=64, context_lens=lens, scale=1 / math.sqrt(192.0))
    out, cache, dq, kw = _mla_sinks_case(cuda, w, np.full(128, -np.inf, np.float32), fused, 0)
    if fused:  # attend again without the append: the cache now holds the new rows
        kw = {}
    plain = paged_decode_mla(dq[:, :, :R], dq[:, :, R:], cache, torch.from_numpy(w.block_tables).to(cuda),
                             torch.from_numpy(w.context_lens).to(cuda), w.scale)
    if fused:
        torch.testing.assert_close(out.float(), plain.float(), atol=2e-2, rtol=1e-2)
    else:
        assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
