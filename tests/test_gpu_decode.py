"""GPU parity of paged decode attention against the float64 oracle.

Tolerance (bf16 output): |got - ref| <= 2e-2 + 1e-2 * |ref| elementwise and
relative L2 error <= 1e-2 (kvcase.ATOL / kvcase.RTOL). Every slot a sequence does not own -- the tail of
its last block and every unowned block -- holds NaN, so any read of a masked
slot would show up as a non-finite output.
"""

import math

import numpy as np
import pytest
import torch

from kvcase import ATOL, bits_of, check_attention, slots_for, to_dev_bits
from oracle import fp8, paged
from wavelet_amd import MLALatentCache, PagedKVCache, paged_decode_gqa, paged_decode_mla, synth

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
NAN16 = np.uint16(0x7FC0)


def _owned_mask(w) -> np.ndarray:
    """[NB, BS] True where some sequence's context covers the slot."""
    own = np.zeros((w.num_blocks, w.block_size), bool)
    for i in range(w.batch):
        pos = np.arange(int(w.context_lens[i]))
        own[w.block_tables[i][pos // w.block_size], pos % w.block_size] = True
    return own


def _bf16_caches(w, tag, std=1.0):
    """Logical [NB, BS, H, D] bf16 bit caches, NaN outside every context."""
    shape = (w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim)
    k = synth.normal_bf16(synth.stream_key(w.name, tag, "k"), shape, std=std)
    v = synth.normal_bf16(synth.stream_key(w.name, tag, "v"), shape, std=std)
    own = _owned_mask(w)
    k[~own] = NAN16
    v[~own] = NAN16
    return k, v


def _to_physical(k_log: np.ndarray, v_log: np.ndarray):
    nb, bs, h, d = k_log.shape
    x = 16 // k_log.dtype.itemsize
    kp = np.ascontiguousarray(k_log.reshape(nb, bs, h, d // x, x).transpose(0, 2, 3, 1, 4))
    vp = np.ascontiguousarray(v_log.transpose(0, 2, 3, 1))
    return kp, vp


def _run_gqa(w, cuda, k_log, v_log, q_bits, *, partition_size=0, max_seq_len=None):
    cache = PagedKVCache(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, device=cuda)
    kp, vp = _to_physical(k_log, v_log)
    cache.k.copy_(to_dev_bits(kp, BF16, cuda))
    cache.v.copy_(to_dev_bits(vp, BF16, cuda))
    out = paged_decode_gqa(
        to_dev_bits(q_bits, BF16, cuda), cache, torch.from_numpy(w.block_tables).to(cuda),
        torch.from_numpy(w.context_lens).to(cuda), w.scale, partition_size=partition_size,
        max_seq_len=max_seq_len,
    )
    return paged.bf16_to_f32(bits_of(out))


def _gqa_case(w, cuda, tag="a", partition_size=0, q_std=1.0, kv_std=1.0):
    k, v = _bf16_caches(w, tag, std=kv_std)
    q = synth.normal_bf16(synth.stream_key(w.name, tag, "q"), (w.batch, w.num_q_heads, w.head_dim), std=q_std)
    got = _run_gqa(w, cuda, k, v, q, partition_size=partition_size)
    kf, vf = paged.bf16_to_f32(k), paged.bf16_to_f32(v)
    qf = paged.bf16_to_f32(q)
    ref = paged.decode_gqa(qf, kf, vf, w.block_tables, w.context_lens, w.scale)
    ref_bf16 = paged.decode_gqa(qf, kf, vf, w.block_tables, w.context_lens, w.scale, p_bf16=True)
    a, r = check_attention(got, ref, f"{w.name} P={partition_size}")
    ra, rr = paged.max_abs_and_rel(paged.bf16_to_f32(paged.f32_to_bf16(ref_bf16.astype(np.float32))), ref)
    print(f"{w.name} P={partition_size}: gpu err abs {a:.2e} rel {r:.2e} | reference bf16 path abs {ra:.2e} rel {rr:.2e}")


def test_decode_qwen25_05b_shape(cuda):
    """14 q / 2 kv heads, d=64, block 16, batch 128, contexts U{256..2048}; Q/K/V ~ N(0,1)/8."""
    w = synth.qwen25_05b_workload()
    _gqa_case(w, cuda, q_std=1 / 8, kv_std=1 / 8)


def test_decode_qwen3_4b_shape_fixed_4096(cuda):
    """32 q / 8 kv heads, d=128, block 16, context 4096 (batch reduced to 8 for the oracle)."""
    w = synth.qwen3_4b_workload(batch=8)
    _gqa_case(w, cuda)


def test_decode_qwen3_4b_shape_variable_lengths(cuda):
    w = synth.qwen3_4b_workload(batch=6, context=None)
    for p in (0, 512):
        _gqa_case(w, cuda, partition_size=p)


# Qwen3-4B, Qwen2.5-0.5B, Qwen2.5-7B, 16 heads on one KV head, GPT-OSS-like, Qwen3-30B-A3B, Qwen3-0.6B
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (28, 4, 128), (16, 1, 128), (8, 8, 64), (32, 4, 128),
                                     (16, 8, 128)])
def test_decode_edge_lengths_and_partitions(cuda, hq, hkv, d):
    lens = np.array([0, 1, 2, 15, 16, 17, 63, 255, 256, 257, 700, 1024])
    w = synth.make_decode_workload(f"edge{hq}x{hkv}x{d}", batch=len(lens), num_kv_heads=hkv, num_q_heads=hq,
                                   head_dim=d, block_size=16, context_lens=lens)
    for p in (16, 64, 256, 0):
        _gqa_case(w, cuda, tag=f"p{p}", partition_size=p)


def test_decode_block_size_64(cuda):
    lens = np.array([1, 64, 65, 500, 2048])
    w = synth.make_decode_workload("bs64", batch=len(lens), num_kv_heads=4, num_q_heads=16, head_dim=128,
                                   block_size=64, context_lens=lens)
    _gqa_case(w, cuda, partition_size=128)


def test_decode_reference_ignore_slot_known_answer(cuda):
    """The reference's sigmoid(0.625)*[2,-1] answer with NaN in every never-read slot."""
    from test_oracle import ignore_slot_case

    kc, vc, q, bt, lens, scale, expected = ignore_slot_case()
    w = synth.DecodeWorkload("ignore", num_blocks=2, block_size=16, num_kv_heads=1, num_q_heads=1, head_dim=64,
                             context_lens=lens.astype(np.int32), block_tables=bt, scale=scale)
    got = _run_gqa(w, cuda, paged.f32_to_bf16(kc), paged.f32_to_bf16(vc), paged.f32_to_bf16(q))
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, expected, atol=1e-2, rtol=0)


def test_decode_fp8_rollout_groups(cuda):
    """Qwen2.5-7B shape groups (28 q / 4 kv, d=128), fp8 KV: 4 groups x 8 sharing a 1024-token prompt.

    The cache is filled through the fp8 append path (prompt once per group in
    whole-block runs, then each member's private tokens, then this step's
    token) and checked bit-exact; attention reads the shared prompt blocks
    from every member's block table.
    """
    w = synth.qwen25_7b_group_workload(num_groups=4)
    H, D, BS, NB = w.num_kv_heads, w.head_dim, w.block_size, w.num_blocks
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint8)
    ks = np.zeros((NB, H), np.float32)
    vs = np.zeros((NB, H), np.float32)
    cache = PagedKVCache(NB, BS, H, D, kv_dtype="fp8_e4m3", device=cuda)

    ctx = w.context_lens.astype(np.int64)
    lo = np.where(np.arange(w.batch) % w.group_size == 0, 0, w.prefix_len)  # prompt written by member 0 only
    steps = [("fill", slots_for(w, lo, ctx - 1)), ("new", w.new_token_slots())]
    for name, sl in steps:
        kb = synth.normal_bf16(synth.stream_key(w.name, name, "k"), (len(sl), H, D))
        vb = synth.normal_bf16(synth.stream_key(w.name, name, "v"), (len(sl), H, D))
        paged.append_fp8(kc, vc, ks, vs, kb, vb, sl)
        cache.append(to_dev_bits(kb, BF16, cuda), to_dev_bits(vb, BF16, cuda), torch.from_numpy(sl).to(cuda))
    assert np.array_equal(bits_of(cache.k), kc) and np.array_equal(bits_of(cache.v), vc)
    np.testing.assert_array_equal(cache.k_scale.cpu().numpy(), ks)
    np.testing.assert_array_equal(cache.v_scale.cpu().numpy(), vs)

    q = synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, w.num_q_heads, D))
    out = paged_decode_gqa(to_dev_bits(q, BF16, cuda), cache, torch.from_numpy(w.block_tables).to(cuda),
                           torch.from_numpy(w.context_lens).to(cuda), w.scale)
    got = paged.bf16_to_f32(bits_of(out))
    k_log = paged.k_logical(kc).reshape(NB, BS, H, D)
    v_log = paged.v_logical(vc)
    kf = fp8.dequantize(k_log, ks[:, None, :, None])
    vf = fp8.dequantize(v_log, vs[:, None, :, None])
    ref = paged.decode_gqa(paged.bf16_to_f32(q), kf, vf, w.block_tables, w.context_lens, w.scale)
    a, r = check_attention(got, ref, "fp8 groups")
    print(f"fp8 groups: err abs {a:.2e} rel {r:.2e}")


def _mla_case(cuda, lens, heads=128, bs=64, partition_size=0, tag="m"):
    R, P = 512, 64
    w = synth.make_decode_workload(f"mla{tag}", batch=len(lens), num_kv_heads=1, num_q_heads=heads,
                                   head_dim=R + P, block_size=bs, context_lens=np.asarray(lens),
                                   scale=1 / math.sqrt(192.0))
    own = _owned_mask(w)
    lat = synth.normal_bf16(synth.stream_key(w.name, "lat"), (w.num_blocks, bs, R + P))
    lat[~own] = NAN16
    q = synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, heads, R + P))
    cache = MLALatentCache(w.num_blocks, bs, R, P, device=cuda)
    cache.latent.copy_(to_dev_bits(lat, BF16, cuda))
    dq = to_dev_bits(q, BF16, cuda)
    out = paged_decode_mla(dq[:, :, :R], dq[:, :, R:], cache, torch.from_numpy(w.block_tables).to(cuda),
                           torch.from_numpy(w.context_lens).to(cuda), w.scale, partition_size=partition_size)
    got = paged.bf16_to_f32(bits_of(out))
    ref = paged.decode_mla(paged.bf16_to_f32(q), paged.bf16_to_f32(lat), w.block_tables, w.context_lens, w.scale)
    a, r = check_attention(got, ref, f"mla {tag}")
    print(f"mla {tag}: err abs {a:.2e} rel {r:.2e}")


def test_decode_mla_deepseek_v3_shape(cuda):
    """128 heads over a 512+64 latent, block 64, context 4096 (batch reduced to 4 for the oracle)."""
    _mla_case(cuda, [4096, 4096, 4096, 4096], tag="dsv3")


@pytest.mark.parametrize("heads", [16, 32, 64, 128])
def test_decode_mla_edge_lengths(cuda, heads):
    for p in (64, 0):
        _mla_case(cuda, [0, 1, 17, 64, 65, 300, 1000], heads=heads, partition_size=p, tag=f"edge{heads}p{p}")


@pytest.mark.parametrize("heads,partition", [(128, 64), (128, 0), (16, 32), (64, 160)])
def test_decode_mla_batches_of_eight(cuda, heads, partition):
    """Batches of 8 and 16 take the launch that puts every partition of a sequence on one XCD
    (item k is sequence k mod 8 + 8 (k / 8 / P), partition k / 8 mod P): ragged lengths make the
    partition counts differ between sequences, so a wrong sequence or partition index either
    attends the wrong tokens or leaves a partial unwritten."""
    lens = [0, 1, 17, 64, 65, 300, 1000, 4096]
    _mla_case(cuda, lens, heads=heads, partition_size=partition, tag=f"b8h{heads}p{partition}")
    _mla_case(cuda, lens[::-1] + [33, 2047, 96, 7, 640, 1, 128, 3000], heads=heads, partition_size=partition,
              tag=f"b16h{heads}p{partition}")


@pytest.mark.parametrize("bs,partition", [(16, 32), (16, 0), (64, 96), (32, 160), (128, 32), (256, 96), (256, 0)])
def test_decode_mla_block_sizes_and_partitions(cuda, bs, partition):
    """32-token steps that straddle two blocks, partitions that start inside a block,
    and tails that end inside a step (NaN in every slot no sequence owns)."""
    _mla_case(cuda, [5, 31, 32, 33, 95, 96, 97, 333, 1024, 2047], bs=bs, partition_size=partition,
              tag=f"bs{bs}p{partition}")


@pytest.mark.parametrize("heads,bs,partition,nseq",
                         [(128, 64, 0, 10), (16, 64, 96, 10), (64, 16, 32, 10), (32, 32, 0, 10), (128, 64, 64, 16),
                          (128, 256, 0, 16), (32, 128, 160, 10)])
def test_fused_mla_append_decode_equals_append_then_decode(cuda, heads, bs, partition, nseq):
    """One launch (latent append + MLA attention) leaves the cache bit-identical to
    wkv_mla_append and attends within tolerance of the separate path and of the oracle; the new
    token's slot and every unowned slot hold NaN before the step, so attending the new token from
    the cache instead of its inputs, or reading past the context, shows up as NaN. A batch of 16
    takes the launch that keeps the partitions of a sequence on one XCD."""
    R, P = 512, 64
    lens = np.array([1, 2, 31, 32, 33, 64, 65, 300, 1024, 1025, 3, 96, 97, 700, 2000, 129][:nseq])
    w = synth.make_decode_workload(f"fusedmla{heads}{bs}{partition}n{nseq}", batch=len(lens), num_kv_heads=1,
                                   num_q_heads=heads, head_dim=R + P, block_size=bs, context_lens=lens,
                                   scale=1 / math.sqrt(192.0))
    own = _owned_mask(w)
    ctx = w.context_lens.astype(np.int64)
    new_slots = w.new_token_slots()
    lat = synth.normal_bf16(synth.stream_key(w.name, "lat"), (w.num_blocks, bs, R + P))
    lat[~own] = NAN16
    lat.reshape(-1, R + P)[new_slots] = NAN16  # the appended token is not in the cache yet
    caches = [MLALatentCache(w.num_blocks, bs, R, P, device=cuda) for _ in range(2)]
    for c in caches:
        c.latent.copy_(to_dev_bits(lat, BF16, cuda))
    kvc_bits = synth.normal_bf16(synth.stream_key(w.name, "kvc"), (w.batch, R))
    kpe_bits = synth.normal_bf16(synth.stream_key(w.name, "kpe"), (w.batch, P))
    kvc, kpe = to_dev_bits(kvc_bits, BF16, cuda), to_dev_bits(kpe_bits, BF16, cuda)
    q_bits = synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, heads, R + P))
    q = to_dev_bits(q_bits, BF16, cuda)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    slots = torch.from_numpy(new_slots).to(cuda)
    caches[0].append(kvc, kpe, slots)
    ref_out = paged_decode_mla(q[:, :, :R], q[:, :, R:], caches[0], bt, sl, w.scale, partition_size=partition)
    out = paged_decode_mla(q[:, :, :R], q[:, :, R:], caches[1], bt, sl, w.scale, partition_size=partition,
                           new_kv_c=kvc, new_k_pe=kpe, slot_mapping=slots)
    torch.cuda.synchronize()
    assert torch.equal(caches[0].latent.view(torch.int16), caches[1].latent.view(torch.int16)), "latent differs"
    torch.testing.assert_close(out.float(), ref_out.float(), atol=2e-2, rtol=1e-2)
    full = lat.copy()
    full.reshape(-1, R + P)[new_slots, :R] = kvc_bits
    full.reshape(-1, R + P)[new_slots, R:] = kpe_bits
    ref = paged.decode_mla(paged.bf16_to_f32(q_bits), paged.bf16_to_f32(full), w.block_tables, ctx, w.scale)
    a, r = check_attention(paged.bf16_to_f32(bits_of(out)), ref, f"fused mla {heads}")
    print(f"fused mla heads={heads} bs={bs} P={partition}: err abs {a:.2e} rel {r:.2e}")


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
@pytest.mark.parametrize("hq,hkv,d,bs", [(32, 8, 128, 16), (14, 2, 64, 16), (16, 4, 128, 64), (32, 8, 128, 32),
                                         (14, 2, 64, 128), (8, 2, 128, 256), (32, 4, 128, 16), (16, 8, 128, 16)])
def test_fused_append_decode_equals_append_then_decode(cuda, kv_dtype, hq, hkv, d, bs, shared):
    """One launch (append + attention) leaves the cache bit-identical to wkv_append(_fp8) and
    attends within tolerance (bf16 attends the new token from its inputs, a different summation
    order; fp8 reads it back from the cache, so there the outputs are bit-identical too). Both
    read policies (``shared``: K/V kept cached, else streamed), one-workgroup and merged plans."""
    lens = np.array([1, 2, 16, 17, 64, 65, 300, 1024, 1025, 2000])
    w = synth.make_decode_workload(f"fused{kv_dtype}{hq}{bs}", batch=len(lens), num_kv_heads=hkv, num_q_heads=hq,
                                   head_dim=d, block_size=bs, context_lens=lens)
    fp8 = kv_dtype == "fp8_e4m3"
    caches = [PagedKVCache(w.num_blocks, bs, hkv, d, kv_dtype=kv_dtype, device=cuda) for _ in range(2)]
    ctx = w.context_lens.astype(np.int64)
    pslots = slots_for(w, np.zeros(w.batch, np.int64), ctx - 1)
    kp = synth.normal_bf16(synth.stream_key(w.name, "pk"), (len(pslots), hkv, d))
    vp = synth.normal_bf16(synth.stream_key(w.name, "pv"), (len(pslots), hkv, d))
    for c in caches:
        c.append(to_dev_bits(kp, BF16, cuda), to_dev_bits(vp, BF16, cuda), torch.from_numpy(pslots).to(cuda))
    nslots = torch.from_numpy(w.new_token_slots()).to(cuda)
    kn = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "nk"), (w.batch, hkv, d), std=4.0), BF16, cuda)
    vn = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "nv"), (w.batch, hkv, d), std=4.0), BF16, cuda)
    q_bits = synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, hq, d))
    q = to_dev_bits(q_bits, BF16, cuda)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    for p in (0, 4 * bs):
        caches[0].append(kn, vn, nslots)
        ref_out = paged_decode_gqa(q, caches[0], bt, sl, w.scale, partition_size=p, shared_blocks=shared)
        out = paged_decode_gqa(q, caches[1], bt, sl, w.scale, partition_size=p, new_key=kn, new_value=vn,
                               slot_mapping=nslots, shared_blocks=shared)
        torch.cuda.synchronize()
        assert torch.equal(caches[0].k.view(torch.uint8), caches[1].k.view(torch.uint8)), f"K differs (P={p})"
        assert torch.equal(caches[0].v.view(torch.uint8), caches[1].v.view(torch.uint8)), f"V differs (P={p})"
        if fp8:
            assert torch.equal(caches[0].k_scale, caches[1].k_scale) and torch.equal(caches[0].v_scale, caches[1].v_scale)
        if fp8:
            assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), f"output differs (P={p})"
        else:
            torch.testing.assert_close(out.float(), ref_out.float(), atol=2e-2, rtol=1e-2,
                                       msg=lambda m: f"fused vs separate (P={p}): {m}")
    # and against the oracle on the final cache contents
    gk, gv = caches[1].gather(bt, sl, dequant=fp8)
    kf = paged.bf16_to_f32(bits_of(gk))
    vf = paged.bf16_to_f32(bits_of(gv))
    # gathered contexts are contiguous: attend sequence by sequence
    ref = np.zeros((w.batch, hq, d))
    g = hq // hkv
    cu = np.concatenate([[0], np.cumsum(w.context_lens)])
    qf = paged.bf16_to_f32(q_bits).astype(np.float64)
    for i in range(w.batch):
        kk, vv = kf[cu[i]:cu[i + 1]].astype(np.float64), vf[cu[i]:cu[i + 1]].astype(np.float64)
        for h in range(hkv):
            s = qf[i, h * g:(h + 1) * g] @ kk[:, h].T * w.scale
            pr = np.exp(s - s.max(axis=1, keepdims=True))
            pr /= pr.sum(axis=1, keepdims=True)
            ref[i, h * g:(h + 1) * g] = pr @ vv[:, h]
    # the new tokens are drawn with std 4 (so that mishandling them shows): outputs and their bf16
    # rounding scale with them
    check_attention(paged.bf16_to_f32(bits_of(out)), ref, f"fused {kv_dtype}", abs_bound=4 * ATOL)


def test_decode_matches_golden_output(cuda, golden_dir):
    from golden import make_golden as mg

    w, k, v, q = mg.gqa_decode_case()
    got = _run_gqa(w, cuda, k, v, q)
    check_attention(got, np.load(golden_dir / "gqa_decode.npz")["out"], "golden gqa")


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
def test_grpo_group_decode_with_block_manager(cuda, kv_dtype, shared):
    """A GRPO group end to end: one prompt (partial last block) shared by 8 members through the
    block manager, copy-on-write of the shared partial block, three fused decode steps; caches
    bit-exact against the oracle's, attention within tolerance, under both read policies."""
    from wavelet_amd import BlockManager

    H, HQ, D, BS, NB = 4, 28, 128, 16, 256
    is_fp8 = kv_dtype == "fp8_e4m3"
    m = BlockManager(NB, BS)
    group = [f"m{j}" for j in range(8)]
    prompt_len = 1000
    m.allocate(group[0], np.arange(prompt_len), cache_salt="policy-3")
    for g in group[1:]:
        m.fork(group[0], g)
    npdt = np.uint8 if is_fp8 else np.uint16
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=npdt)
    ks = np.zeros((NB, H), np.float32)
    vs = np.zeros((NB, H), np.float32)
    cache = PagedKVCache(NB, BS, H, D, kv_dtype=kv_dtype, device=cuda)
    blocks = np.array(m.blocks_of(group[0]), np.int64)
    pos = np.arange(prompt_len)
    pslots = blocks[pos // BS] * BS + pos % BS
    kp = synth.normal_bf16(synth.stream_key("grpo", kv_dtype, "pk"), (prompt_len, H, D))
    vp = synth.normal_bf16(synth.stream_key("grpo", kv_dtype, "pv"), (prompt_len, H, D))
    if is_fp8:
        paged.append_fp8(kc, vc, ks, vs, kp, vp, pslots)
    else:
        paged.append_bf16(kc, vc, kp, vp, pslots)
    cache.append(to_dev_bits(kp, BF16, cuda), to_dev_bits(vp, BF16, cuda), torch.from_numpy(pslots).to(cuda))
    scale = 1 / math.sqrt(D)
    for step in range(3):
        slots, cow = m.append_slots(group)
        assert (len(cow) == 7) == (step == 0)  # only the first write into the shared partial block copies
        if cow:
            pairs = np.array(cow, np.int64)
            cache.copy_blocks(torch.from_numpy(pairs).to(cuda))
            for s_, d_ in pairs:
                kc[d_], vc[d_], ks[d_], vs[d_] = kc[s_], vc[s_], ks[s_], vs[s_]
        bt, lens = m.tables(group)
        kn = synth.normal_bf16(synth.stream_key("grpo", kv_dtype, step, "k"), (8, H, D))
        vn = synth.normal_bf16(synth.stream_key("grpo", kv_dtype, step, "v"), (8, H, D))
        q = synth.normal_bf16(synth.stream_key("grpo", kv_dtype, step, "q"), (8, HQ, D))
        if is_fp8:
            paged.append_fp8(kc, vc, ks, vs, kn, vn, slots)
        else:
            paged.append_bf16(kc, vc, kn, vn, slots)
        out = paged_decode_gqa(to_dev_bits(q, BF16, cuda), cache, torch.from_numpy(bt).to(cuda),
                               torch.from_numpy(lens).to(cuda), scale, new_key=to_dev_bits(kn, BF16, cuda),
                               new_value=to_dev_bits(vn, BF16, cuda), slot_mapping=torch.from_numpy(slots).to(cuda),
                               shared_blocks=shared)
        assert np.array_equal(bits_of(cache.k), kc) and np.array_equal(bits_of(cache.v), vc), f"cache step {step}"
        if is_fp8:
            np.testing.assert_array_equal(cache.k_scale.cpu().numpy(), ks)
            kf = fp8.dequantize(paged.k_logical(kc).reshape(NB, BS, H, D), ks[:, None, :, None])
            vf = fp8.dequantize(paged.v_logical(vc), vs[:, None, :, None])
        else:
            kl, vl = paged.logical_kv(kc, vc)
            kf, vf = paged.bf16_to_f32(kl), paged.bf16_to_f32(vl)
        ref = paged.decode_gqa(paged.bf16_to_f32(q), kf, vf, bt, lens, scale)
        check_attention(paged.bf16_to_f32(bits_of(out)), ref, f"grpo {kv_dtype} step {step}")


@pytest.mark.parametrize("fused,partition", [(False, 0), (True, 0), (False, 1024), (True, 1024)])
def test_decode_mla_score_spikes_restart_partitions(cuda, fused, partition):
    """Scores that jump far above a partition's first-step maximum.

    Every head attends the same query here and two latent rows point along it
    (steps 3 and 20 of the first 1024 tokens, ~90 and ~80 log2-units above
    everything before them): the online softmax must move its reference twice
    within one 1024-token partition, or once in each of two partitions with
    the library's partition (96 tokens here), and the output must still match
    the float64 oracle."""
    R, P, H, BS = 512, 64, 128, 64
    lens = np.array([1500, 4096, 700])
    w = synth.make_decode_workload(f"mlaspike{int(fused)}{partition}", batch=len(lens), num_kv_heads=1, num_q_heads=H,
                                   head_dim=R + P, block_size=BS, context_lens=lens, scale=1 / math.sqrt(192.0))
    own = _owned_mask(w)
    lat = paged.bf16_to_f32(synth.normal_bf16(synth.stream_key(w.name, "lat"), (w.num_blocks, BS, R + P)))
    q0 = paged.bf16_to_f32(synth.normal_bf16(synth.stream_key(w.name, "q0"), (R + P,)))
    unit = q0 / np.linalg.norm(q0)
    for i in range(w.batch):
        for pos, mag in ((3 * 32 + 5, 40.0), (20 * 32 + 7, 72.0)):
            if pos < lens[i] - 1:
                blk = w.block_tables[i][pos // BS]
                lat[blk, pos % BS] = unit * mag
    lat_bits = paged.f32_to_bf16(lat)
    lat_bits[~own] = NAN16
    q = np.broadcast_to(q0, (w.batch, H, R + P)).copy()
    q_bits = paged.f32_to_bf16(q)
    cache = MLALatentCache(w.num_blocks, BS, R, P, device=cuda)
    cache.latent.copy_(to_dev_bits(lat_bits, BF16, cuda))
    dq = to_dev_bits(q_bits, BF16, cuda)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    full = lat_bits.copy()
    if fused:
        slots = w.new_token_slots()
        kv = synth.normal_bf16(synth.stream_key(w.name, "kv"), (w.batch, R + P))
        full.reshape(-1, R + P)[slots] = kv
        out = paged_decode_mla(dq[:, :, :R], dq[:, :, R:], cache, bt, sl, w.scale,
                               new_kv_c=to_dev_bits(np.ascontiguousarray(kv[:, :R]), BF16, cuda),
                               new_k_pe=to_dev_bits(np.ascontiguousarray(kv[:, R:]), BF16, cuda),
                               slot_mapping=torch.from_numpy(slots).to(cuda), partition_size=partition)
    else:
        out = paged_decode_mla(dq[:, :, :R], dq[:, :, R:], cache, bt, sl, w.scale, partition_size=partition)
    got = paged.bf16_to_f32(bits_of(out))
    ref = paged.decode_mla(paged.bf16_to_f32(q_bits), paged.bf16_to_f32(full), w.block_tables, w.context_lens,
                           w.scale)
    # the spike rows dominate: outputs are ~72/|q0| * q0 (entries up to ~15), whose bf16 rounding is 2^-9 relative
    a, r = check_attention(got, ref, f"mla spikes fused={fused} P={partition}", abs_bound=8 * ATOL)
    print(f"mla spikes fused={fused} P={partition}: err abs {a:.2e} rel {r:.2e}")
