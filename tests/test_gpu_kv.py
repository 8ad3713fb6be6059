"""GPU parity of append / gather / block copy against the oracle: bit-exact.

Every cache byte and every gathered element is compared, with untouched slots
pre-poisoned (NaN bit patterns) so a stray write or read shows up.
"""

import numpy as np
import pytest
import torch

from kvcase import bits_of, slots_for, to_dev_bits
from oracle import paged
from wavelet_amd import MLALatentCache, PagedKVCache, synth

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _upload(cache: PagedKVCache, kc: np.ndarray, vc: np.ndarray, ks=None, vs=None) -> None:
    dt = BF16 if kc.dtype == np.uint16 else torch.uint8
    cache.k.copy_(to_dev_bits(kc, dt, cache.device))
    cache.v.copy_(to_dev_bits(vc, dt, cache.device))
    if ks is not None:
        cache.k_scale.copy_(torch.from_numpy(ks))
        cache.v_scale.copy_(torch.from_numpy(vs))


def _assert_cache_equal(cache: PagedKVCache, kc, vc, ks=None, vs=None, what=""):
    gk, gv = bits_of(cache.k), bits_of(cache.v)
    assert np.array_equal(gk, kc), f"{what}: K cache differs at {np.argwhere(gk != kc)[:5].tolist()}"
    assert np.array_equal(gv, vc), f"{what}: V cache differs at {np.argwhere(gv != vc)[:5].tolist()}"
    if ks is not None:
        np.testing.assert_array_equal(cache.k_scale.cpu().numpy().view(np.uint32), ks.view(np.uint32))
        np.testing.assert_array_equal(cache.v_scale.cpu().numpy().view(np.uint32), vs.view(np.uint32))


def test_append_then_gather_bf16_32_seqs_bit_exact(cuda):
    """1 layer, 8 KV heads x 128, block 16, 32 seqs with lengths U{1..512}, 2048 blocks."""
    w = synth.append_gather_workload()
    H, D, BS, NB = w.num_kv_heads, w.head_dim, w.block_size, w.num_blocks
    kc, vc = paged.empty_cache(NB, BS, H, D, fill=0xFFFF)
    cache = PagedKVCache(NB, BS, H, D, device=cuda)
    _upload(cache, kc, vc)

    ctx = w.context_lens.astype(np.int64)
    # cached context, written as one prefill append
    pslots = slots_for(w, np.zeros(w.batch, np.int64), ctx - 1)
    kp = synth.normal_bf16(synth.stream_key(w.name, "prefill_k"), (len(pslots), H, D))
    vp = synth.normal_bf16(synth.stream_key(w.name, "prefill_v"), (len(pslots), H, D))
    paged.append_bf16(kc, vc, kp, vp, pslots)
    cache.append(to_dev_bits(kp, BF16, cuda), to_dev_bits(vp, BF16, cuda), torch.from_numpy(pslots).to(cuda))
    _assert_cache_equal(cache, kc, vc, what="prefill")

    # decode append: one token per sequence, padded with slot -1 entries, and
    # key/value taken as strided views of a fused qkv buffer
    nslots = w.new_token_slots()
    nslots = np.insert(nslots, [3, 10, 10], -1)
    T = len(nslots)
    qkv = synth.normal_bf16(synth.stream_key(w.name, "qkv"), (T, 48, D))  # 32 q + 8 k + 8 v heads
    kn, vn = qkv[:, 32:40], qkv[:, 40:48]
    paged.append_bf16(kc, vc, kn, vn, nslots)
    dqkv = to_dev_bits(qkv, BF16, cuda)
    cache.append(dqkv[:, 32:40], dqkv[:, 40:48], torch.from_numpy(nslots).to(cuda))
    _assert_cache_equal(cache, kc, vc, what="decode append")

    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    gk, gv = cache.gather(bt, sl)
    ok, ov = paged.gather(kc, vc, w.block_tables, w.context_lens)
    np.testing.assert_array_equal(bits_of(gk), ok)
    np.testing.assert_array_equal(bits_of(gv), ov)
    # and the gather is the inverse of the appends
    assert not np.any(ok == 0xFFFF)


@pytest.mark.parametrize("H,D,BS,T", [(8, 128, 16, 1000), (2, 64, 64, 777), (4, 128, 32, 256), (3, 64, 16, 300),
                                       (8, 128, 16, 255)])
def test_append_bf16_many_tokens_shuffled_slots_bit_exact(cuda, H, D, BS, T):
    """Prompt-sized appends (the transposing kernel from 256 tokens on, the per-chunk one below):
    slots in random order across blocks, every 7th token skipped (-1), a ragged last window,
    key/value as strided views of a fused buffer; untouched slots keep their poison."""
    NB = (2 * T + BS - 1) // BS
    rng = np.random.default_rng(T * 31 + D)
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    slots[::7] = -1
    kc, vc = paged.empty_cache(NB, BS, H, D, fill=0xFFFF)
    cache = PagedKVCache(NB, BS, H, D, device=cuda)
    _upload(cache, kc, vc)
    qkv = synth.normal_bf16(synth.stream_key("bulk", str(T), str(D)), (T, 3 * H, D))
    paged.append_bf16(kc, vc, qkv[:, H:2 * H], qkv[:, 2 * H:], slots)
    d = to_dev_bits(qkv, BF16, cuda)
    cache.append(d[:, H:2 * H], d[:, 2 * H:], torch.from_numpy(slots).to(cuda))
    _assert_cache_equal(cache, kc, vc, what=f"bulk append T={T}")


@pytest.mark.parametrize("H,D,BS", [(8, 128, 16), (2, 64, 32), (3, 128, 64)])
def test_append_bf16_prompt_runs_bit_exact(cuda, H, D, BS):
    """Prompt-shaped appends through the transposing kernel: each sequence's tokens at
    consecutive positions of its blocks (a random block order), continuing cached contexts of
    0, 8, 3, 13, 21 tokens (8-token groups that start aligned, mid-group and mid-block), one
    skipped token (-1) and a ragged end: the 16-byte V stores of aligned groups and the
    per-token stores of the others, bit-exact against the oracle."""
    rng = np.random.default_rng(BS * 7 + D)
    ctx = [0, 8, 3, 13, 21]
    new = [300, 77, 129, 64, 250]
    per_seq = [-(-(c + n) // BS) for c, n in zip(ctx, new)]
    NB = sum(per_seq) + 4
    order = rng.permutation(NB)
    slots, used = [], 0
    for c, n, nb in zip(ctx, new, per_seq):
        blocks = order[used:used + nb]
        used += nb
        pos = np.arange(c, c + n)
        slots.append(blocks[pos // BS].astype(np.int64) * BS + pos % BS)
    slots = np.concatenate(slots)
    slots[101] = -1
    T = len(slots)
    assert T >= 256  # the transposing kernel's range
    kc, vc = paged.empty_cache(NB, BS, H, D, fill=0xFFFF)
    cache = PagedKVCache(NB, BS, H, D, device=cuda)
    _upload(cache, kc, vc)
    kv = synth.normal_bf16(synth.stream_key("prompt-runs", str(BS), str(D)), (T, 2 * H, D))
    paged.append_bf16(kc, vc, kv[:, :H], kv[:, H:], slots)
    d = to_dev_bits(kv, BF16, cuda)
    cache.append(d[:, :H], d[:, H:], torch.from_numpy(slots).to(cuda))
    _assert_cache_equal(cache, kc, vc, what=f"prompt runs BS={BS} D={D}")


def _exhaustive_bf16_rows(h: int, d: int) -> np.ndarray:
    """All 65,536 bf16 patterns sorted by magnitude (NaN last), as [tokens, h, d]."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = paged.bf16_to_f32(bits)
    key = np.where(np.isnan(vals), np.inf, np.abs(vals))
    order = np.argsort(key, kind="stable")
    return bits[order].reshape(-1, h, d)


@pytest.mark.parametrize("BS", [16, 32])
def test_append_fp8_bulk_runs(cuda, BS):
    """Prompt-sized fp8 appends (the bulk kernel): runs that continue partly filled blocks with
    growing scales, fresh blocks, runs across 64-token windows, skipped slots between runs,
    shuffled block order -- bit-exact codes and scales."""
    NB, H, D = 256, 2, 128
    rng = np.random.default_rng(BS)
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint8, fill=0xAA)
    ks = np.zeros((NB, H), np.float32)
    vs = np.zeros((NB, H), np.float32)
    cache = PagedKVCache(NB, BS, H, D, kv_dtype="fp8_e4m3", device=cuda)
    _upload(cache, kc, vc, ks, vs)

    def both(key_bits, val_bits, slots, what):
        assert len(slots) >= 64  # the bulk kernel's range
        paged.append_fp8(kc, vc, ks, vs, key_bits, val_bits, slots)
        cache.append(to_dev_bits(key_bits, BF16, cuda), to_dev_bits(val_bits, BF16, cuda),
                     torch.from_numpy(np.asarray(slots, np.int64)).to(cuda))
        _assert_cache_equal(cache, kc, vc, ks, vs, what=what)

    blocks = rng.permutation(NB)[:120]
    fill = rng.integers(1, BS, 40)
    s1 = np.concatenate([b * BS + np.arange(f) for b, f in zip(blocks[:40], fill)]).astype(np.int64)
    both(synth.normal_bf16(synth.stream_key("fp8bulk", BS, "k1"), (len(s1), H, D), std=0.01),
         synth.normal_bf16(synth.stream_key("fp8bulk", BS, "v1"), (len(s1), H, D), std=0.02), s1, "partial fills")
    parts = [b * BS + np.arange(f, min(BS, f + int(rng.integers(1, BS)))) for b, f in zip(blocks[:40], fill)]
    parts += [b * BS + np.arange(int(rng.integers(1, BS + 1))) for b in blocks[40:]]
    order = rng.permutation(len(parts))
    s2 = []
    for i in order:
        s2.append(parts[i])
        if rng.random() < 0.3:
            s2.append(np.full(int(rng.integers(1, 4)), -1))
    s2 = np.concatenate(s2).astype(np.int64)
    both(synth.normal_bf16(synth.stream_key("fp8bulk", BS, "k2"), (len(s2), H, D), std=5.0),
         synth.normal_bf16(synth.stream_key("fp8bulk", BS, "v2"), (len(s2), H, D), std=50.0), s2,
         "continued and fresh runs")


def test_append_fp8_bulk_whole_blocks_every_pattern(cuda):
    """Whole fresh 16-token blocks through the bulk kernel (its fast path: 16-byte stores, the
    hardware code conversion) holding every bf16 pattern -- sorted by magnitude, so blocks span
    subnormals to infinities, then shuffled, so NaN lands in most blocks (which must take the
    general path) -- plus a block whose tokens come in reverse slot order: codes and scales
    bit-exact against the oracle."""
    NB, BS, H, D = 128, 16, 2, 128
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint8, fill=0xAA)
    ks = np.zeros((NB, H), np.float32)
    vs = np.zeros((NB, H), np.float32)
    cache = PagedKVCache(NB, BS, H, D, kv_dtype="fp8_e4m3", device=cuda)
    _upload(cache, kc, vc, ks, vs)

    def both(key_bits, val_bits, slots, what):
        assert len(slots) >= 64  # the bulk kernel's range
        paged.append_fp8(kc, vc, ks, vs, key_bits, val_bits, slots)
        cache.append(to_dev_bits(key_bits, BF16, cuda), to_dev_bits(val_bits, BF16, cuda),
                     torch.from_numpy(np.asarray(slots, np.int64)).to(cuda))
        _assert_cache_equal(cache, kc, vc, ks, vs, what=what)

    rows = _exhaustive_bf16_rows(H, D)  # [256, 2, 128]
    whole = np.arange(256, dtype=np.int64)  # blocks 0..15, offsets 0..15 in order
    both(rows, rows[::-1].copy(), whole, "sorted patterns in whole blocks")
    rng = np.random.default_rng(7)
    mixed = rows.reshape(-1)[rng.permutation(rows.size)].reshape(rows.shape)
    both(mixed, mixed[::-1].copy(), whole + 16 * BS, "shuffled patterns in whole blocks")
    rev = (32 * BS + np.arange(BS)[::-1]).astype(np.int64)  # one block, tokens in reverse slot order
    fwd = np.arange(33 * BS, 37 * BS, dtype=np.int64)
    both(rows[:80], rows[80:160].copy(), np.concatenate([rev, fwd]), "a block in reverse order")


def test_append_fp8_bit_exact_exhaustive_and_scale_growth(cuda):
    NB, BS, H, D = 512, 16, 2, 128
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint8, fill=0xAA)
    ks = np.zeros((NB, H), np.float32)
    vs = np.zeros((NB, H), np.float32)
    cache = PagedKVCache(NB, BS, H, D, kv_dtype="fp8_e4m3", device=cuda)
    _upload(cache, kc, vc, ks, vs)

    def both(key_bits, val_bits, slots, what):
        paged.append_fp8(kc, vc, ks, vs, key_bits, val_bits, slots)
        cache.append(to_dev_bits(key_bits, BF16, cuda), to_dev_bits(val_bits, BF16, cuda),
                     torch.from_numpy(np.asarray(slots, np.int64)).to(cuda))
        _assert_cache_equal(cache, kc, vc, ks, vs, what=what)

    # 1) every bf16 pattern, one fresh block per token (runs of one at offset 0)
    rows = _exhaustive_bf16_rows(H, D)  # [256, 2, 128]
    slots = np.arange(rows.shape[0], dtype=np.int64) * BS
    both(rows, rows[::-1].copy(), slots, "exhaustive")

    # 2) prefill runs: 3 sequences, whole and partial blocks, mixed magnitudes
    pre = np.concatenate([np.arange(300 * BS, 300 * BS + 40), np.arange(320 * BS, 320 * BS + 16),
                          np.arange(330 * BS, 330 * BS + 5)]).astype(np.int64)
    xk = synth.normal_bf16(synth.stream_key("fp8gpu", "pk"), (len(pre), H, D), std=3.0)
    xv = synth.normal_bf16(synth.stream_key("fp8gpu", "pv"), (len(pre), H, D), std=0.01)
    both(xk, xv, pre, "prefill runs")

    # 3) decode appends into partial blocks with growing / shrinking magnitudes:
    #    scale growth re-encodes earlier entries (subnormal rounding included)
    for step, mag in enumerate([0.5, 60.0, 1e-3, 9000.0, 2.0]):
        sl = np.array([300 * BS + 40 + step, 330 * BS + 5 + step, -1], np.int64)
        k = synth.normal_bf16(synth.stream_key("fp8gpu", "dk", step), (3, H, D), std=mag)
        v = synth.normal_bf16(synth.stream_key("fp8gpu", "dv", step), (3, H, D), std=mag * 3)
        both(k, v, sl, f"decode step {step}")

    # gather: raw codes and exact bf16 dequantisation
    bt = np.array([[300, 301, 302], [320, 0, 0], [330, 0, 0]], np.int32)
    lens = np.array([45, 16, 10], np.int32)
    dbt, dl = torch.from_numpy(bt).to(cuda), torch.from_numpy(lens).to(cuda)
    gk, gv = cache.gather(dbt, dl)
    ok, ov = paged.gather(kc, vc, bt, lens)
    np.testing.assert_array_equal(bits_of(gk), ok)
    np.testing.assert_array_equal(bits_of(gv), ov)
    qk, qv = cache.gather(dbt, dl, dequant=True)
    ek = paged.f32_to_bf16(paged.dequant_gathered(ok, ks, bt, lens, BS))
    ev = paged.f32_to_bf16(paged.dequant_gathered(ov, vs, bt, lens, BS))
    np.testing.assert_array_equal(bits_of(qk), ek)
    np.testing.assert_array_equal(bits_of(qv), ev)


def test_copy_blocks_copies_kv_and_scales(cuda):
    NB, BS, H, D = 64, 16, 4, 64
    for dtype in ("bf16", "fp8_e4m3"):
        fp8 = dtype == "fp8_e4m3"
        npdt = np.uint8 if fp8 else np.uint16
        kc = synth.random_u64(synth.stream_key("cp", dtype, "k"), NB * H * D * BS).astype(npdt)
        vc = synth.random_u64(synth.stream_key("cp", dtype, "v"), NB * H * D * BS).astype(npdt)
        x = 16 if fp8 else 8
        kc = kc.reshape(NB, H, D // x, BS, x)
        vc = vc.reshape(NB, H, D, BS)
        ks = np.arange(NB * H, dtype=np.float32).reshape(NB, H)
        vs = -ks
        cache = PagedKVCache(NB, BS, H, D, kv_dtype=dtype, device=cuda)
        _upload(cache, kc, vc, ks if fp8 else None, vs if fp8 else None)
        mapping = np.array([[3, 10], [7, 11], [3, 12], [40, 2]], np.int64)
        cache.copy_blocks(torch.from_numpy(mapping).to(cuda))
        for s, d in mapping:
            kc[d], vc[d], ks[d], vs[d] = kc[s], vc[s], ks[s], vs[s]
        _assert_cache_equal(cache, kc, vc, ks if fp8 else None, vs if fp8 else None, what=f"copy {dtype}")


def test_mla_append_bit_exact(cuda):
    NB, BS, R, P = 32, 64, 512, 64
    lat = np.full((NB, BS, R + P), 0xFFFF, np.uint16)
    cache = MLALatentCache(NB, BS, R, P, device=cuda)
    cache.latent.copy_(to_dev_bits(lat, BF16, cuda))
    slots = np.array([0, 65, -1, 2047, 700, 1000], np.int64)
    kvc = synth.normal_bf16(synth.stream_key("mla_app", "c"), (len(slots), R))
    kpe = synth.normal_bf16(synth.stream_key("mla_app", "p"), (len(slots), P))
    for t, s in enumerate(slots):
        if s >= 0:
            lat[s // BS, s % BS, :R] = kvc[t]
            lat[s // BS, s % BS, R:] = kpe[t]
    cache.append(to_dev_bits(kvc, BF16, cuda), to_dev_bits(kpe, BF16, cuda), torch.from_numpy(slots).to(cuda))
    np.testing.assert_array_equal(bits_of(cache.latent), lat)


def test_append_gather_matches_golden_digests(cuda, golden_dir):
    """The committed fixture: cache and gathered context digests after prefill + decode append."""
    import json

    from golden import make_golden as mg

    w, pslots, kp, vp, nslots, kn, vn = mg.append_gather_case()
    expected = json.loads((golden_dir / "outputs.json").read_text())["append_gather"]
    assert synth.sha256_of(w.block_tables, w.context_lens, pslots, kp, vp, nslots, kn, vn) == expected["inputs"]
    H, D, BS, NB = w.num_kv_heads, w.head_dim, w.block_size, w.num_blocks
    kc, vc = paged.empty_cache(NB, BS, H, D, fill=0xFFFF)
    cache = PagedKVCache(NB, BS, H, D, device=cuda)
    _upload(cache, kc, vc)
    for sl, k, v in ((pslots, kp, vp), (nslots, kn, vn)):
        cache.append(to_dev_bits(k, BF16, cuda), to_dev_bits(v, BF16, cuda), torch.from_numpy(sl).to(cuda))
    assert synth.sha256_of(bits_of(cache.k)) == expected["k_cache"]
    assert synth.sha256_of(bits_of(cache.v)) == expected["v_cache"]
    gk, gv = cache.gather(torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda))
    assert synth.sha256_of(bits_of(gk)) == expected["gathered_k"]
    assert synth.sha256_of(bits_of(gv)) == expected["gathered_v"]


def _fp8_case(cuda, NB, BS, H, D):
    kc, vc = paged.empty_cache(NB, BS, H, D, dtype=np.uint8, fill=0xAA)
    ks = np.zeros((NB, H), np.float32)
    vs = np.zeros((NB, H), np.float32)
    cache = PagedKVCache(NB, BS, H, D, kv_dtype="fp8_e4m3", device=cuda)
    _upload(cache, kc, vc, ks, vs)

    def both(key_bits, val_bits, slots, what):
        paged.append_fp8(kc, vc, ks, vs, key_bits, val_bits, slots)
        cache.append(to_dev_bits(key_bits, BF16, cuda), to_dev_bits(val_bits, BF16, cuda),
                     torch.from_numpy(np.asarray(slots, np.int64)).to(cuda))
        _assert_cache_equal(cache, kc, vc, ks, vs, what=what)
    return both


def test_append_fp8_decode_shaped_call(cuda):
    """One token per sequence (a decode step's append, 256 one-token runs in scattered,
    partly filled blocks; most scales grow and re-encode the block's earlier codes): the
    bulk kernel's many-runs-per-window case, bit-exact codes and scales."""
    NB, BS, H, D = 512, 16, 4, 128
    rng = np.random.default_rng(11)
    both = _fp8_case(cuda, NB, BS, H, D)
    blocks = rng.permutation(NB)[:256]
    fill = rng.integers(1, BS, 256)
    prior = np.concatenate([b * BS + np.arange(f) for b, f in zip(blocks, fill)]).astype(np.int64)
    both(synth.normal_bf16(synth.stream_key("fp8dec", "k0"), (len(prior), H, D), std=0.05),
         synth.normal_bf16(synth.stream_key("fp8dec", "v0"), (len(prior), H, D), std=0.05), prior, "contexts")
    step = (blocks * BS + fill).astype(np.int64)
    step[::17] = -1  # sequences without a token this step
    both(synth.normal_bf16(synth.stream_key("fp8dec", "k1"), (256, H, D), std=2.0),
         synth.normal_bf16(synth.stream_key("fp8dec", "v1"), (256, H, D), std=0.01), step, "decode step")


@pytest.mark.parametrize("BS", [16, 32])
def test_append_fp8_prompt_sized_call(cuda, BS):
    """A prompt-sized call (4,096 tokens or more: the bulk kernel's prompt launch shape):
    several prompts in shuffled blocks, one continuing a partly filled block, one ending in a
    partial block -- bit-exact codes and scales."""
    NB, H, D = 1024 // (BS // 16), 2, 128
    rng = np.random.default_rng(BS + 3)
    both = _fp8_case(cuda, NB, BS, H, D)
    blocks = rng.permutation(NB)
    head = (blocks[0] * BS + np.arange(5)).astype(np.int64)  # a block already holding 5 tokens
    both(synth.normal_bf16(synth.stream_key("fp8pr", BS, "k0"), (64, H, D), std=0.01),
         synth.normal_bf16(synth.stream_key("fp8pr", BS, "v0"), (64, H, D), std=0.01),
         np.concatenate([head, np.full(59, -1)]), "a partly filled block")
    lens = [BS - 5 + 7 * BS, 1500, 1111, 1000, 700]  # the first continues blocks[0]
    slots = [np.concatenate([blocks[0] * BS + np.arange(5, BS), blocks[1:8].repeat(BS) * BS + np.tile(np.arange(BS), 7)])]
    nb = 8
    for L in lens[1:]:
        k = (L + BS - 1) // BS
        own = blocks[nb:nb + k]
        nb += k
        slots.append((own.repeat(BS) * BS + np.tile(np.arange(BS), k))[:L])
    s = np.concatenate(slots).astype(np.int64)
    assert len(s) >= 4096
    both(synth.normal_bf16(synth.stream_key("fp8pr", BS, "k1"), (len(s), H, D), std=1.0),
         synth.normal_bf16(synth.stream_key("fp8pr", BS, "v1"), (len(s), H, D), std=3.0), s, "prompts")
