"""GPU parity of the group-aware (GRPO) decode against the plain decode and the float64 oracle.

Groups are built the way the engine builds them: one prompt allocated through
``BlockManager`` and forked to every member (shared physical blocks), private
generated tokens per member, then a decode step whose append copies a still
shared partially filled block first (copy-on-write). ``prefix_lens`` comes from
``BlockManager.shared_prefix_tokens``. The grouped call reads the prompt with
another cache policy than the members' own tokens but over the same tiles, so
it must equal the plain call on the same inputs bit for bit (attention only,
and fused with the step's append: outputs and cache), in any dispatch order
(batch order, ``grouped_decode_order``), and match the oracle. Unowned bf16
slots hold NaN, so a read outside any context would surface.
"""

import math

import numpy as np
import pytest
import torch

from kvcase import bits_of, check_attention, to_dev_bits
from oracle import fp8, paged
from wavelet_amd import (BlockManager, PagedKVCache, decode_plan, grouped_decode_order, paged_decode_gqa,
                         paged_decode_gqa_grouped, synth)

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _build_groups(n_groups, gs, BS, NB, prompt_lens, gen_lens):
    """Block tables of n_groups GRPO groups after prompt + generated tokens: (manager, ids)."""
    m = BlockManager(NB, BS, enable_prefix_caching=False)
    ids = [(g, j) for g in range(n_groups) for j in range(gs)]
    for g in range(n_groups):
        m.allocate((g, 0), np.arange(int(prompt_lens[g])) + 7919 * g)
        for j in range(1, gs):
            m.fork((g, 0), (g, j))
    # generated tokens, one decode step at a time (copy-on-write of shared partial blocks)
    for step in range(int(max(gen_lens))):
        m.append_slots([s for k, s in enumerate(ids) if gen_lens[k] > step])
    return m, ids


def _fill(m, ids, BS, NB, H, D, prompt_lens, tag, is_fp8, skip_last=0):
    """Cache contents (numpy, physical layout) holding every sequence's tokens
    (all but the last `skip_last`): prompt token p of group g is P_g[p] wherever
    it is stored; generated tokens are private. Copy-on-write copies carry the
    prompt tokens they duplicate."""
    slot_val = {}
    for (g, j) in ids:
        blocks = m.blocks_of((g, j))
        for pos in range(m.seq_len((g, j)) - skip_last):
            slot = blocks[pos // BS] * BS + pos % BS
            key = ("p", g, pos) if pos < prompt_lens[g] else ("s", g, j, pos)
            assert slot_val.setdefault(slot, key) == key, "two different tokens in one slot"
    slots = np.array(sorted(slot_val), np.int64)
    keys = [slot_val[s] for s in slots]
    kb = np.stack([synth.normal_bf16(synth.stream_key(tag, "k", *k), (H, D)) for k in keys])
    vb = np.stack([synth.normal_bf16(synth.stream_key(tag, "v", *k), (H, D)) for k in keys])
    if is_fp8:
        kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint8)
        ks = np.zeros((NB, H), np.float32)
        vs = np.zeros((NB, H), np.float32)
        paged.append_fp8(kc, vc, ks, vs, kb, vb, slots)
        return kc, vc, ks, vs
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint16, fill=0x7FC0)
    paged.append_bf16(kc, vc, kb, vb, slots)
    return kc, vc, None, None


def _upload(cache, kc, vc, ks, vs, cuda):
    dt = torch.uint8 if kc.dtype == np.uint8 else BF16
    cache.k.copy_(to_dev_bits(kc, dt, cuda).view(cache.k.dtype))
    cache.v.copy_(to_dev_bits(vc, dt, cuda).view(cache.v.dtype))
    if ks is not None:
        cache.k_scale.copy_(torch.from_numpy(ks).to(cuda))
        cache.v_scale.copy_(torch.from_numpy(vs).to(cuda))


def _oracle(q_bits, kc, vc, ks, vs, bt, lens, scale, NB, BS, H, D):
    if ks is not None:
        kf = fp8.dequantize(paged.k_logical(kc).reshape(NB, BS, H, D), ks[:, None, :, None])
        vf = fp8.dequantize(paged.v_logical(vc), vs[:, None, :, None])
    else:
        kl, vl = paged.logical_kv(kc, vc)
        kf, vf = paged.bf16_to_f32(kl), paged.bf16_to_f32(vl)
    return paged.decode_gqa(paged.bf16_to_f32(q_bits), kf, vf, bt, lens, scale)


CASES = [
    # hq, hkv, d, bs, groups, group size, prompt lengths, max generated
    (28, 4, 128, 16, 3, 8, (1024, 1000, 17), 70),   # Qwen2.5-7B heads, 56 rows per group
    (14, 2, 64, 16, 3, 4, (300, 16, 5), 40),        # d=64, short prompts
    (32, 8, 128, 16, 2, 3, (257, 512), 33),         # 24 rows
    (16, 1, 128, 64, 1, 16, (700,), 20),            # 256 rows per group: 16 row tiles, 4 workgroups
    (8, 8, 64, 16, 5, 1, (40, 64, 1, 200, 90), 9),  # groups of one
    (28, 4, 128, 32, 2, 8, (1024, 500), 100),       # block 32, a prompt ending mid-block
    (16, 2, 128, 128, 2, 4, (600, 129), 50),        # block 128
]


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
@pytest.mark.parametrize("hq,hkv,d,bs,n_groups,gs,prompts,max_gen", CASES)
def test_grouped_decode_matches_plain_and_oracle(cuda, kv_dtype, hq, hkv, d, bs, n_groups, gs, prompts, max_gen):
    is_fp8 = kv_dtype == "fp8_e4m3"
    tag = f"grp{kv_dtype}{hq}{hkv}{d}{bs}{gs}"
    NB = 2048 if bs == 16 else 512
    gen = synth.randint(synth.stream_key(tag, "gen"), n_groups * gs, 0, max_gen)
    m, ids = _build_groups(n_groups, gs, bs, NB, prompts, gen)
    # this step's token: copy-on-write first, as the engine would
    new_slots, _ = m.append_slots(ids)
    bt, lens = m.tables(ids)
    # the cache before this step's append (tables already include the new token's block)
    kc, vc, ks, vs = _fill(m, ids, bs, NB, hkv, d, prompts, tag, is_fp8, skip_last=1)
    pre = np.array([m.shared_prefix_tokens([(g, j) for j in range(gs)]) for g in range(n_groups)], np.int32)
    assert pre.max() > 0
    caches = [PagedKVCache(NB, bs, hkv, d, kv_dtype=kv_dtype, device=cuda) for _ in range(3)]
    for c in caches:
        _upload(c, kc, vc, ks, vs, cuda)
    scale = 1 / math.sqrt(d)
    B = len(ids)
    q_bits = synth.normal_bf16(synth.stream_key(tag, "q"), (B, hq, d))
    kn_bits = synth.normal_bf16(synth.stream_key(tag, "nk"), (B, hkv, d))
    vn_bits = synth.normal_bf16(synth.stream_key(tag, "nv"), (B, hkv, d))
    q, kn, vn = (to_dev_bits(x, BF16, cuda) for x in (q_bits, kn_bits, vn_bits))
    dbt, dlens = torch.from_numpy(bt).to(cuda), torch.from_numpy(lens).to(cuda)
    dslots, dpre = torch.from_numpy(new_slots).to(cuda), torch.from_numpy(pre).to(cuda)

    for p in (0, 2 * bs):
        # attention only, before the step's token: lengths without it
        lens0 = dlens - 1
        plain = paged_decode_gqa(q, caches[0], dbt, lens0, scale, partition_size=p)
        grouped = paged_decode_gqa_grouped(q, caches[0], dbt, lens0, dpre, gs, scale, partition_size=p)
        assert torch.equal(grouped.view(torch.int16), plain.view(torch.int16)), f"grouped vs plain (P={p})"
        order = grouped_decode_order(lens0, gs, hkv, int(lens0.max()), bs, p)
        ordered = paged_decode_gqa_grouped(q, caches[0], dbt, lens0, dpre, gs, scale, partition_size=p,
                                           seq_order=order)
        assert torch.equal(ordered.view(torch.int16), plain.view(torch.int16)), f"grouped, ordered (P={p})"
        # the whole step, fused: the grouped call appends into caches[1], the plain one into caches[2]
        if p == 0:
            caches[0].append(kn, vn, dslots)
            ref_out = paged_decode_gqa(q, caches[0], dbt, dlens, scale)
            out = paged_decode_gqa_grouped(q, caches[1], dbt, dlens, dpre, gs, scale, new_key=kn, new_value=vn,
                                           slot_mapping=dslots)
            plain_fused = paged_decode_gqa(q, caches[2], dbt, dlens, scale, new_key=kn, new_value=vn,
                                           slot_mapping=dslots)
            torch.cuda.synchronize()
            for c in (caches[1], caches[2]):
                assert torch.equal(caches[0].k.view(torch.uint8), c.k.view(torch.uint8)), "K differs"
                assert torch.equal(caches[0].v.view(torch.uint8), c.v.view(torch.uint8)), "V differs"
                if is_fp8:
                    assert torch.equal(caches[0].k_scale, c.k_scale)
                    assert torch.equal(caches[0].v_scale, c.v_scale)
            assert torch.equal(out.view(torch.int16), plain_fused.view(torch.int16)), "grouped fused vs plain fused"
            torch.testing.assert_close(out.float(), ref_out.float(), atol=2e-2, rtol=1e-2,
                                       msg=lambda s: f"grouped fused vs append + plain: {s}")
    # oracle on the final cache (after the append)
    if is_fp8:
        paged.append_fp8(kc, vc, ks, vs, kn_bits, vn_bits, new_slots)
    else:
        paged.append_bf16(kc, vc, kn_bits, vn_bits, new_slots)
    assert np.array_equal(bits_of(caches[1].k), kc) and np.array_equal(bits_of(caches[1].v), vc)
    ref = _oracle(q_bits, kc, vc, ks, vs, bt, lens, scale, NB, bs, hkv, d)
    a, r = check_attention(paged.bf16_to_f32(bits_of(out)), ref, f"grouped {kv_dtype} {hq}/{hkv}")
    print(f"grouped {kv_dtype} hq={hq} hkv={hkv} d={d} gs={gs}: err abs {a:.2e} rel {r:.2e}")


def test_grouped_decode_prefix_claims(cuda):
    """prefix_lens of 0 (no sharing used), below the shared blocks, unaligned, and above the
    shortest member all give the plain result bit for bit (they steer the read policy only)."""
    hq, hkv, d, bs, gs = 28, 4, 128, 16, 8
    tag = "grpclaims"
    NB = 1024
    prompts = (600, 333)
    gen = synth.randint(synth.stream_key(tag, "gen"), 2 * gs, 0, 50)
    m, ids = _build_groups(2, gs, bs, NB, prompts, gen)
    bt, lens = m.tables(ids)
    kc, vc, _, _ = _fill(m, ids, bs, NB, hkv, d, prompts, tag, False)
    cache = PagedKVCache(NB, bs, hkv, d, device=cuda)
    _upload(cache, kc, vc, None, None, cuda)
    q_bits = synth.normal_bf16(synth.stream_key(tag, "q"), (len(ids), hq, d))
    q = to_dev_bits(q_bits, BF16, cuda)
    dbt, dlens = torch.from_numpy(bt).to(cuda), torch.from_numpy(lens).to(cuda)
    scale = 1 / math.sqrt(d)
    plain = paged_decode_gqa(q, cache, dbt, dlens, scale)
    shared = [m.shared_prefix_tokens([(g, j) for j in range(gs)]) for g in range(2)]
    for claim in ([0, 0], [100, 37], [shared[0], shared[1]], [shared[0] - 5, 1]):
        pre = torch.tensor(claim, dtype=torch.int32, device=cuda)
        got = paged_decode_gqa_grouped(q, cache, dbt, dlens, pre, gs, scale)
        assert torch.equal(got.view(torch.int16), plain.view(torch.int16)), f"claim {claim}"
    ref = _oracle(q_bits, kc, vc, None, None, bt, lens, scale, NB, bs, hkv, d)
    check_attention(paged.bf16_to_f32(bits_of(got)), ref, "grouped claims")


def test_grouped_decode_ragged_last_group_and_empty(cuda):
    """batch not a multiple of group_size, a zero-length sequence and a one-token one."""
    hq, hkv, d, bs, gs = 16, 4, 128, 16, 4
    tag = "grpragged"
    NB = 512
    m = BlockManager(NB, bs, enable_prefix_caching=False)
    ids = list(range(10))
    prompts = {0: 64, 4: 33, 8: 1}
    for g0 in (0, 4, 8):
        m.allocate(g0, np.arange(prompts[g0]))
        for j in range(g0 + 1, min(g0 + gs, 10)):
            m.fork(g0, j)
    for _ in range(20):
        m.append_slots([1, 2, 5, 9])
    bt, lens = m.tables(ids)
    lens[3] = 0  # an empty member (its table is still the group's)
    kc, vc = paged.empty_cache(NB, bs, hkv, d, dtype=np.uint16, fill=0x7FC0)
    for sid in ids:
        blocks = m.blocks_of(sid)
        pos = np.arange(m.seq_len(sid))
        sl = np.array(blocks, np.int64)[pos // bs] * bs + pos % bs
        g0 = sid // gs * gs
        kb = np.stack([synth.normal_bf16(synth.stream_key(tag, "k", g0 if p < prompts[g0] else sid, p), (hkv, d))
                       for p in pos])
        vb = np.stack([synth.normal_bf16(synth.stream_key(tag, "v", g0 if p < prompts[g0] else sid, p), (hkv, d))
                       for p in pos])
        paged.append_bf16(kc, vc, kb, vb, sl)
    cache = PagedKVCache(NB, bs, hkv, d, device=cuda)
    _upload(cache, kc, vc, None, None, cuda)
    q_bits = synth.normal_bf16(synth.stream_key(tag, "q"), (10, hq, d))
    q = to_dev_bits(q_bits, BF16, cuda)
    dbt, dlens = torch.from_numpy(bt).to(cuda), torch.from_numpy(lens).to(cuda)
    pre = torch.tensor([64, 33, 1], dtype=torch.int32, device=cuda)
    scale = 1 / math.sqrt(d)
    got = paged_decode_gqa_grouped(q, cache, dbt, dlens, pre, gs, scale, partition_size=32)
    plain = paged_decode_gqa(q, cache, dbt, dlens, scale, partition_size=32)
    assert torch.equal(got.view(torch.int16), plain.view(torch.int16))
    assert torch.count_nonzero(got[3]) == 0  # empty context: zeros
    ref = _oracle(q_bits, kc, vc, None, None, bt, lens, scale, NB, bs, hkv, d)
    check_attention(paged.bf16_to_f32(bits_of(got)), ref, "grouped ragged")


def _expected_grouped_order(lens, gs, hkv, max_seq, bs, partition):
    """The order's definition: classes of whole groups (group g in class g % n), n the
    number of XCD classes of the launch (8 / gcd(8, chunks * Hkv), 1 when the classes
    would be unequal); stable longest-first within a class; rank r of class c at r*n + c."""
    _, _, chunks = decode_plan(len(lens), hkv, max_seq, bs, partition)
    n = 8 // math.gcd(8, chunks * hkv)
    if len(lens) % (gs * n):
        n = 1
    out = np.empty(len(lens), np.int64)
    for c in range(n):
        idx = np.array([i for i in range(len(lens)) if (i // gs) % n == c])
        ranked = idx[np.argsort(-lens[idx].astype(np.int64), kind="stable")]
        out[np.arange(len(ranked)) * n + c] = ranked
    return out, n


@pytest.mark.parametrize("batch,gs,hkv,max_seq,part,n_cls", [
    (256, 8, 4, 4096, 0, 2),   # Qwen2.5-7B groups: one workgroup per (sequence, KV head)
    (48, 3, 1, 1000, 0, 8),    # one KV head: eight classes
    (64, 4, 2, 2000, 128, 2),  # two chunks per sequence
    (44, 3, 1, 1000, 0, 1),    # eight classes would be unequal: the plain longest-first order
    (40, 5, 8, 4096, 0, 1),    # eight KV heads: a head already stays on one XCD
])
def test_grouped_decode_order(cuda, batch, gs, hkv, max_seq, part, n_cls):
    rng = np.random.default_rng(batch + gs)
    lens = rng.integers(0, max_seq + 1, batch).astype(np.int32)
    lens[: batch // 4] = lens[0]  # ties
    want, n = _expected_grouped_order(lens, gs, hkv, max_seq, 16, part)
    assert n == n_cls
    got = grouped_decode_order(torch.from_numpy(lens).to(cuda), gs, hkv, max_seq, 16, part).cpu().numpy()
    np.testing.assert_array_equal(got, want)
