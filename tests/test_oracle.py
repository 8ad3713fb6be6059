"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against something independent of it: torch's
float8_e4m3fn cast and libm log2 (library routines), torch's
scaled_dot_product_attention in float64, scalar pure-Python re-statements on
small inputs, closed forms, and the reference's own known answer
(tests/test_deepseek_attention.py:100-118 in the reference).
"""

import math

import numpy as np
import pytest
import torch

from oracle import fp8, paged
from wavelet_amd import synth


def _torch_e4m3(x32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x32.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encode_all_bf16_patterns_match_torch():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = paged.bf16_to_f32(bits)
    np.testing.assert_array_equal(fp8.e4m3_encode(x), _torch_e4m3(x))


def test_e4m3_encode_random_fp32_patterns_match_torch():
    u = synth.random_u64(synth.stream_key("oracle", "fp32bits"), 1 << 20).astype(np.uint64)
    x = (u & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    # plus a dense sweep of the e4m3 range where rounding decisions happen
    sweep = np.linspace(-500.0, 500.0, 200001, dtype=np.float32)
    tiny = np.linspace(-2.0**-5, 2.0**-5, 100001, dtype=np.float32)
    for arr in (x, sweep, tiny):
        np.testing.assert_array_equal(fp8.e4m3_encode(arr), _torch_e4m3(arr))


def test_e4m3_decode_matches_torch_table():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = fp8.e4m3_decode(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


def _torch_pow2_scale(a: np.ndarray) -> np.ndarray:
    # The reference expression (attention.py:42-48) evaluated by torch / libm.
    t = torch.from_numpy(a.astype(np.float32))
    return torch.exp2(torch.ceil(torch.log2(t.clamp_min(1e-10) / 448.0))).numpy()


def test_pow2_scale_matches_reference_expression_for_every_bf16_amax():
    bits = np.arange(0, 0x7F80, dtype=np.uint16)  # all non-negative finite bf16
    a = paged.bf16_to_f32(bits)
    np.testing.assert_array_equal(fp8.pow2_scale(a), _torch_pow2_scale(a))


def test_pow2_scale_invariants():
    a = np.abs(synth.normal(synth.stream_key("oracle", "amax"), 100000)).astype(np.float32) * 37.0
    a = np.concatenate([a, np.float32(448.0) * np.exp2(np.arange(-30, 30)).astype(np.float32)])
    s = fp8.pow2_scale(a).astype(np.float64)
    m, _ = np.frexp(s)
    assert np.all(m == 0.5), "scale must be a power of two"
    r = np.maximum(a, 1e-10).astype(np.float64) / 448.0
    assert np.all(s >= r * (1 - 2**-23)) and np.all(s < 2 * r * (1 + 2**-23))
    # amax/s lands in (224, 448]: no clamp ever bites for finite inputs
    q = a / s
    assert np.all(q <= 448.0 * (1 + 2**-22))


def test_quantize_matches_reference_roundtrip_convention():
    x = (synth.normal(synth.stream_key("oracle", "q"), 4096) * 3.0).astype(np.float32).reshape(32, 128)
    amax = np.abs(x).max(axis=1)
    s = fp8.pow2_scale(amax)[:, None]
    got = fp8.dequantize(fp8.quantize(x, s), s)
    t = torch.from_numpy(x)
    scale = torch.exp2(torch.ceil(torch.log2(t.abs().amax(-1, keepdim=True).clamp_min(1e-10) / 448.0)))
    ref = ((t / scale).clamp(-448, 448).to(torch.float8_e4m3fn).float() * scale).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# append / gather

def _kv_inputs(w, tag):
    n = w.batch
    k = synth.normal_bf16(synth.stream_key(w.name, tag, "k"), (n, w.num_kv_heads, w.head_dim))
    v = synth.normal_bf16(synth.stream_key(w.name, tag, "v"), (n, w.num_kv_heads, w.head_dim))
    return k, v


def test_append_gather_round_trip_bf16():
    w = synth.append_gather_workload(seqs=8, max_len=100, num_blocks=256)
    kc, vc = paged.empty_cache(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim)
    total = int(w.context_lens.sum())
    # write every token position of every sequence
    kk = synth.normal_bf16(synth.stream_key("rt", "k"), (total, w.num_kv_heads, w.head_dim))
    vv = synth.normal_bf16(synth.stream_key("rt", "v"), (total, w.num_kv_heads, w.head_dim))
    slots = []
    for i, L in enumerate(w.context_lens):
        pos = np.arange(L)
        slots.append(w.block_tables[i][pos // w.block_size].astype(np.int64) * w.block_size + pos % w.block_size)
    slots = np.concatenate(slots)
    before_k = kc.copy()
    paged.append_bf16(kc, vc, kk, vv, slots)
    gk, gv = paged.gather(kc, vc, w.block_tables, w.context_lens)
    np.testing.assert_array_equal(gk, kk)
    np.testing.assert_array_equal(gv, vv)
    # blocks no sequence owns are untouched
    used = set(slots // w.block_size)
    free = [b for b in range(w.num_blocks) if b not in used]
    np.testing.assert_array_equal(kc[free], before_k[free])


def test_append_bf16_matches_elementwise_loop_and_skips_padding():
    nb, bs, h, d = 6, 16, 2, 64
    kc, vc = paged.empty_cache(nb, bs, h, d)
    rng_k = synth.normal_bf16(synth.stream_key("tiny", "k"), (5, h, d))
    rng_v = synth.normal_bf16(synth.stream_key("tiny", "v"), (5, h, d))
    slots = np.array([17, -1, 3, 95, 40], dtype=np.int64)
    paged.append_bf16(kc, vc, rng_k, rng_v, slots)
    ek = np.zeros((nb, h, d // 8, bs, 8), np.uint16)
    ev = np.zeros((nb, h, d, bs), np.uint16)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        b, o = divmod(int(s), bs)
        for hh in range(h):
            for dd in range(d):
                ek[b, hh, dd // 8, o, dd % 8] = rng_k[t, hh, dd]
                ev[b, hh, dd, o] = rng_v[t, hh, dd]
    np.testing.assert_array_equal(kc, ek)
    np.testing.assert_array_equal(vc, ev)


def _scalar_encode(x: float) -> int:
    """Pure-Python e4m3fn encoder (independent of oracle.fp8): RNE, NaN/overflow -> 0x7F."""
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    if math.isnan(x):
        return 0x7F | sign
    a = abs(x)
    if a < 2.0**-6:
        q = round(a * 512.0)  # Python round is half-to-even
        return q | sign
    m, e = math.frexp(a)
    q = round(m * 16.0)
    code = ((e - 1 + 7) << 3) + (q - 8)
    if code >= 0x7F or math.isinf(a):
        code = 0x7F
    return code | sign


def _scalar_decode(c: int) -> float:
    e, m = (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        v = float("nan")
    elif e == 0:
        v = m * 2.0**-9
    else:
        v = (1 + m / 8) * 2.0 ** (e - 7)
    return -v if c & 0x80 else v


def _scalar_scale(amax: float) -> float:
    a = min(max(amax, float(np.float32(1e-10))), float(np.finfo(np.float32).max))
    r = float(np.float32(np.float32(a) / np.float32(448.0)))
    m, e = math.frexp(r)
    return 2.0 ** (e - 1 if m == 0.5 else e)


def _scalar_append_fp8(state, key, value, slots, bs):
    """Per-element pure-Python statement of the fp8 append rule (runs, growth, re-encode)."""
    kcodes, vcodes, kscale, vscale = state  # dicts keyed (blk, off, h, d) / (blk, h)
    t, n = 0, len(slots)
    h, d = key.shape[1], key.shape[2]
    while t < n:
        if slots[t] < 0:
            t += 1
            continue
        blk = slots[t] // bs
        r = 1
        while t + r < n and slots[t + r] >= 0 and slots[t + r] // bs == blk:
            r += 1
        first = slots[t] % bs
        for src, codes, scales in ((key, kcodes, kscale), (value, vcodes, vscale)):
            for hh in range(h):
                vals = [float(src[t + j, hh, dd]) for j in range(r) for dd in range(d)]
                amax = max((abs(v) for v in vals if not math.isnan(v)), default=0.0)
                s_new = _scalar_scale(amax)
                if first == 0:
                    s = s_new
                else:
                    s_old = scales.get((blk, hh), 0.0)
                    s = s_new if s_new > s_old else s_old
                    if s > s_old:
                        for off in range(first):
                            for dd in range(d):
                                c = codes.get((blk, off, hh, dd), 0)
                                codes[(blk, off, hh, dd)] = _scalar_encode(_scalar_decode(c) * (s_old / s))
                for j in range(r):
                    off = slots[t + j] % bs
                    for dd in range(d):
                        x = float(np.float32(src[t + j, hh, dd]) / np.float32(s))
                        if not math.isnan(x):
                            x = min(max(x, -448.0), 448.0)
                        codes[(blk, off, hh, dd)] = _scalar_encode(x)
                scales[(blk, hh)] = s
        t += r


def test_append_fp8_matches_scalar_statement_with_growth_and_subnormals():
    nb, bs, h, d = 4, 16, 2, 64
    kc, vc = paged.empty_cache(nb, bs, h, d, dtype=np.uint8)
    ks = np.zeros((nb, h), np.float32)
    vs = np.zeros((nb, h), np.float32)
    state = ({}, {}, {}, {})
    # call 1: prefill run of 5 tokens into block 2, 1 token into block 0
    # call 2..4: one token each into block 2 with growing magnitude (scale grows,
    #            old entries re-encoded, small ones fall into subnormals)
    calls = [
        (np.array([32, 33, 34, 35, 36, 0], np.int64), 1.0),
        (np.array([37, -1], np.int64), 40.0),
        (np.array([38], np.int64), 0.001),
        (np.array([39, 1], np.int64), 5000.0),
    ]
    for ci, (slots, mag) in enumerate(calls):
        kb = synth.normal_bf16(synth.stream_key("fp8s", ci, "k"), (len(slots), h, d), std=mag)
        vb = synth.normal_bf16(synth.stream_key("fp8s", ci, "v"), (len(slots), h, d), std=mag * 0.5)
        if ci == 0:
            kb[0, 0, 0] = 0x7FC0  # NaN input: encodes to the NaN code, ignored by amax
        paged.append_fp8(kc, vc, ks, vs, kb, vb, slots)
        _scalar_append_fp8(state, paged.bf16_to_f32(kb), paged.bf16_to_f32(vb), list(slots), bs)
    kcodes, vcodes, kscale, vscale = state
    kl, vl = paged.k_logical(kc), paged.v_logical(vc)
    for (blk, off, hh, dd), c in kcodes.items():
        assert kl[blk, off, hh, dd // 16, dd % 16] == c, (blk, off, hh, dd)
    for (blk, off, hh, dd), c in vcodes.items():
        assert vl[blk, off, hh, dd] == c, (blk, off, hh, dd)
    for (blk, hh), s in kscale.items():
        assert ks[blk, hh] == np.float32(s)
    for (blk, hh), s in vscale.items():
        assert vs[blk, hh] == np.float32(s)
    # the growth path actually ran: block 2's scale grew past its prefill value
    assert ks[2, 0] > 2.0**-6


def test_fp8_dequantised_error_bound_without_growth():
    nb, bs, h, d = 8, 16, 4, 128
    kc, vc = paged.empty_cache(nb, bs, h, d, dtype=np.uint8)
    ks = np.zeros((nb, h), np.float32)
    vs = np.zeros((nb, h), np.float32)
    x = synth.normal_bf16(synth.stream_key("fp8b", "x"), (bs, h, d), std=2.0)
    slots = np.arange(3 * bs, 4 * bs, dtype=np.int64)  # one whole-block run
    paged.append_fp8(kc, vc, ks, vs, x, x, slots)
    codes, _ = paged.gather(kc, vc, np.array([[3]], np.int32), np.array([bs]))
    deq = paged.dequant_gathered(codes, ks, np.array([[3]], np.int32), np.array([bs]), bs)
    xf = paged.bf16_to_f32(x)
    s = ks[3][None, :, None]
    # e4m3 has 3 fraction bits: |x - x_hat| <= 2^-4 |x| for normals, <= 2^-10 * s below
    err = np.abs(deq - xf)
    assert np.all(err <= np.maximum(np.abs(xf) * 2.0**-4, s * 2.0**-10) * (1 + 1e-6))


# ---------------------------------------------------------------------------
# attention

def _sdpa_reference(q, k_vals, v_vals, bt, lens, scale):
    """torch SDPA (float64) on the gathered context, GQA by repeating KV heads."""
    b, hq, d = q.shape
    hkv = k_vals.shape[2]
    g = hq // hkv
    out = np.zeros((b, hq, d))
    bs = k_vals.shape[1]
    for i in range(b):
        L = int(lens[i])
        pos = np.arange(L)
        blk = bt[i][pos // bs]
        kk = torch.from_numpy(k_vals[blk, pos % bs].astype(np.float64)).permute(1, 0, 2)  # [Hkv, L, D]
        vv = torch.from_numpy(v_vals[blk, pos % bs].astype(np.float64)).permute(1, 0, 2)
        kk = kk.repeat_interleave(g, 0)
        vv = vv.repeat_interleave(g, 0)
        qq = torch.from_numpy(q[i].astype(np.float64))[:, None, :]  # [Hq, 1, D]
        o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, scale=scale)
        out[i] = o[:, 0, :].numpy()
    return out


def _random_cache_values(w, tag):
    kc = synth.normal_bf16(synth.stream_key(w.name, tag, "kc"), (w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim))
    vc = synth.normal_bf16(synth.stream_key(w.name, tag, "vc"), (w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim))
    return paged.bf16_to_f32(kc), paged.bf16_to_f32(vc)


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128), (28, 4, 128)])
def test_decode_gqa_matches_torch_sdpa(hq, hkv, d):
    w = synth.make_decode_workload(
        f"sdpa{hq}", batch=4, num_kv_heads=hkv, num_q_heads=hq, head_dim=d, block_size=16,
        context_lens=np.array([1, 17, 64, 300]),
    )
    kv, vv = _random_cache_values(w, "a")
    q = paged.bf16_to_f32(synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, hq, d)))
    got = paged.decode_gqa(q, kv, vv, w.block_tables, w.context_lens, w.scale)
    ref = _sdpa_reference(q, kv, vv, w.block_tables, w.context_lens, w.scale)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_decode_gqa_closed_forms():
    w = synth.make_decode_workload("closed", batch=3, num_kv_heads=2, num_q_heads=4, head_dim=64, block_size=16,
                                   context_lens=np.array([1, 40, 40]))
    kv, vv = _random_cache_values(w, "c")
    # sequence 1: all keys identical -> uniform attention -> mean(V)
    bt = w.block_tables
    for pos in range(40):
        kv[bt[1][pos // 16], pos % 16] = kv[bt[1][0], 0]
    # sequence 2: one key aligned with a huge query -> one-hot on that token
    q = paged.bf16_to_f32(synth.normal_bf16(synth.stream_key("closed", "q"), (3, 4, 64)))
    kv[bt[2][1], 5] = 0.0
    kv[bt[2][1], 5, :, 0] = 100.0  # every other key has |k[0]| < 10
    q[2, :, :] = 0.0
    q[2, :, 0] = 1e4
    out = paged.decode_gqa(q, kv, vv, bt, w.context_lens, w.scale)
    np.testing.assert_array_equal(out[0], np.repeat(vv[bt[0][0], 0], 2, axis=0))  # L = 1 -> v0 exactly
    pos = np.arange(40)
    mean_v = vv[bt[1][pos // 16], pos % 16].astype(np.float64).mean(0)
    np.testing.assert_allclose(out[1], np.repeat(mean_v, 2, axis=0), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out[2], np.repeat(vv[bt[2][1], 5], 2, axis=0), rtol=0, atol=1e-12)


def ignore_slot_case():
    """The reference's known answer, restated for a paged decode without sinks.

    tests/test_deepseek_attention.py:100-118: query [0.5, -0.25], one real key
    = value [2, -1], scaling 0.5, a zero-logit zero-value sink, an ignored slot
    holding NaN/inf. Output = sigmoid(0.625) * [2, -1]. Here the sink is a real
    token whose key is 0 (logit 0) and value 0, and every slot past the context
    is poisoned with NaN. head_dim is padded to 64 with zeros.
    """
    nb, bs, h, d = 2, 16, 1, 64
    kc = np.full((nb, bs, h, d), np.nan, np.float32)
    vc = np.full((nb, bs, h, d), np.nan, np.float32)
    kc[1, 0], vc[1, 0] = 0.0, 0.0  # the sink: logit 0, value 0
    kc[1, 1], vc[1, 1] = 0.0, 0.0
    kc[1, 1, 0, :2] = [2.0, -1.0]
    vc[1, 1, 0, :2] = [2.0, -1.0]
    q = np.zeros((1, 1, d), np.float32)
    q[0, 0, :2] = [0.5, -0.25]
    bt = np.array([[1]], np.int32)
    lens = np.array([2], np.int32)
    expected = np.zeros((1, 1, d))
    expected[0, 0, :2] = (1.0 / (1.0 + math.exp(-0.625))) * np.array([2.0, -1.0])
    return kc, vc, q, bt, lens, 0.5, expected


def test_decode_gqa_reference_ignore_slot_known_answer():
    kc, vc, q, bt, lens, scale, expected = ignore_slot_case()
    out = paged.decode_gqa(q, kc, vc, bt, lens, scale)
    assert np.all(np.isfinite(out))
    np.testing.assert_allclose(out, expected, rtol=1e-12, atol=1e-12)


def sink_case():
    """The reference's known answer with its sink passed as a sink.

    tests/test_deepseek_attention.py:100-118: query [0.5, -0.25], one real key
    = value [2, -1], scaling 0.5, a zero-logit zero-value sink (the ``sinks``
    parameter of attention.py:89-95), an ignored slot. Output =
    sigmoid(0.625) * [2, -1]. Here the ignored slot is every slot past the
    one-token context, poisoned with NaN; head_dim is padded to 64 with zeros.
    """
    nb, bs, h, d = 2, 16, 1, 64
    kc = np.full((nb, bs, h, d), np.nan, np.float32)
    vc = np.full((nb, bs, h, d), np.nan, np.float32)
    kc[1, 0], vc[1, 0] = 0.0, 0.0
    kc[1, 0, 0, :2] = [2.0, -1.0]
    vc[1, 0, 0, :2] = [2.0, -1.0]
    q = np.zeros((1, 1, d), np.float32)
    q[0, 0, :2] = [0.5, -0.25]
    bt = np.array([[1]], np.int32)
    lens = np.array([1], np.int32)
    expected = np.zeros((1, 1, d))
    expected[0, 0, :2] = (1.0 / (1.0 + math.exp(-0.625))) * np.array([2.0, -1.0])
    return kc, vc, q, bt, lens, 0.5, np.zeros(1, np.float32), expected


def test_decode_gqa_sink_reference_known_answer():
    kc, vc, q, bt, lens, scale, sinks, expected = sink_case()
    out = paged.decode_gqa(q, kc, vc, bt, lens, scale, sinks=sinks)
    np.testing.assert_allclose(out, expected, rtol=1e-12, atol=1e-12)


def test_decode_gqa_sink_equals_a_zero_value_token():
    """A sink s_h is the same as one more token per sequence whose key scores
    exactly s_h against the query (k = q s_h / (scale |q|^2)) and whose value is
    zero; checked with one query head per KV head so that key can be built."""
    rng = np.random.default_rng(7)
    b, h, d, bs, scale = 5, 3, 64, 16, 0.125
    lens = np.array([0, 1, 17, 40, 33], np.int32)
    nblk = (lens.max() + 1 + bs - 1) // bs
    bt = np.arange(b * nblk, dtype=np.int32).reshape(b, nblk)
    kc = rng.standard_normal((b * nblk, bs, h, d))
    vc = rng.standard_normal((b * nblk, bs, h, d))
    q = rng.standard_normal((b, h, d))
    sinks = np.array([0.7, -2.5, 4.0])
    out = paged.decode_gqa(q, kc, vc, bt, lens, scale, sinks=sinks)
    k2, v2 = kc.copy(), vc.copy()
    for i in range(b):
        pos = lens[i]
        blk, off = bt[i, pos // bs], pos % bs
        for hh in range(h):
            k2[blk, off, hh] = q[i, hh] * (sinks[hh] / (scale * float(q[i, hh] @ q[i, hh])))
            v2[blk, off, hh] = 0.0
    ref = paged.decode_gqa(q, k2, v2, bt, lens + 1, scale)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    assert np.all(out[0] == 0.0)  # no context: the sink takes everything


def test_decode_gqa_sink_closed_forms():
    """-inf sinks change nothing; n identical keys and values under a sink s
    give v * n / (n + e^(s - c)), c the common score."""
    rng = np.random.default_rng(8)
    b, hq, hkv, d, bs, scale = 3, 4, 2, 64, 16, 0.25
    lens = np.array([5, 16, 31], np.int32)
    bt = np.arange(b * 2, dtype=np.int32).reshape(b, 2)
    kc = rng.standard_normal((b * 2, bs, hkv, d))
    vc = rng.standard_normal((b * 2, bs, hkv, d))
    q = rng.standard_normal((b, hq, d))
    none = paged.decode_gqa(q, kc, vc, bt, lens, scale)
    np.testing.assert_array_equal(paged.decode_gqa(q, kc, vc, bt, lens, scale, sinks=np.full(hq, -np.inf)), none)
    kc[:] = kc[0, 0]
    vc[:] = vc[0, 0]
    sinks = np.array([-1.0, 0.0, 2.0, 5.0])
    out = paged.decode_gqa(q, kc, vc, bt, lens, scale, sinks=sinks)
    for i in range(b):
        for h in range(hq):
            c = float(q[i, h] @ kc[0, 0, h // 2]) * scale
            n = float(lens[i])
            np.testing.assert_allclose(out[i, h], vc[0, 0, h // 2] * n / (n + math.exp(sinks[h] - c)), rtol=1e-12)


def test_decode_mla_matches_explicit_non_absorbed_attention():
    """Absorbed MLA == per-head attention with K = W_UK c + rope, V = W_UV c (then W_UV folded out)."""
    rank, rope, hn, heads, dv = 32, 8, 16, 4, 16
    nb, bs, L = 3, 16, 37
    key = synth.stream_key
    c = synth.normal(key("mla", "c"), nb * bs * (rank + rope)).reshape(nb, bs, rank + rope)
    w_uk = synth.normal(key("mla", "wuk"), heads * hn * rank).reshape(heads, hn, rank) / math.sqrt(rank)
    w_uv = synth.normal(key("mla", "wuv"), heads * dv * rank).reshape(heads, dv, rank) / math.sqrt(rank)
    q_nope = synth.normal(key("mla", "qn"), heads * hn).reshape(heads, hn)
    q_pe = synth.normal(key("mla", "qp"), heads * rope).reshape(heads, rope)
    bt = np.array([[2, 0, 1]], np.int32)
    pos = np.arange(L)
    ctx = c[bt[0][pos // bs], pos % bs]  # [L, rank+rope]
    scale = 1.0 / math.sqrt(hn + rope)
    # explicit: per head, k_h = [W_UK c_kv, k_pe], v_h = W_UV c_kv
    explicit = np.zeros((heads, dv))
    for hh in range(heads):
        k_h = np.concatenate([ctx[:, :rank] @ w_uk[hh].T, ctx[:, rank:]], axis=1)
        v_h = ctx[:, :rank] @ w_uv[hh].T
        s = (np.concatenate([q_nope[hh], q_pe[hh]]) @ k_h.T) * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        explicit[hh] = p @ v_h
    # absorbed: q_lat = q_nope W_UK, attend over the latent, then apply W_UV
    q_lat = np.einsum("hn,hnr->hr", q_nope, w_uk)
    q_abs = np.concatenate([q_lat, q_pe], axis=1)[None]
    o_lat = paged.decode_mla(q_abs, c, bt, np.array([L]), scale, kv_lora_rank=rank)[0]
    absorbed = np.einsum("hr,hvr->hv", o_lat, w_uv)
    np.testing.assert_allclose(absorbed, explicit, rtol=1e-10, atol=1e-12)


def test_decode_zero_length_gives_zeros():
    kc = np.zeros((1, 16, 1, 64), np.float32)
    out = paged.decode_gqa(np.ones((1, 2, 64)), kc, kc, np.array([[0]]), np.array([0]), 0.125)
    assert np.all(out == 0)


def _prefill_case(name, hq, hkv, d, bs, qlens, lens):
    w = synth.make_decode_workload(name, batch=len(lens), num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=bs, context_lens=np.asarray(lens))
    kv, vv = _random_cache_values(w, "p")
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int64)
    q = paged.bf16_to_f32(synth.normal_bf16(synth.stream_key(name, "q"), (int(cu[-1]), hq, d)))
    return w, kv, vv, cu, q


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128)])
def test_prefill_gqa_matches_torch_sdpa_with_explicit_mask(hq, hkv, d):
    """Against torch's scaled_dot_product_attention (float64) with the end-aligned causal mask."""
    qlens, lens = [5, 16, 1, 33], [5, 40, 300, 33]  # whole prompt, chunk after context, decode-like, one block+
    w, kv, vv, cu, q = _prefill_case(f"pf{hq}", hq, hkv, d, 16, qlens, lens)
    got = paged.prefill_gqa(q, kv, vv, w.block_tables, w.context_lens, cu, w.scale)
    g = hq // hkv
    for i, (n, length) in enumerate(zip(qlens, lens)):
        pos = np.arange(length)
        blk = w.block_tables[i][pos // 16]
        kk = torch.from_numpy(kv[blk, pos % 16].astype(np.float64)).permute(1, 0, 2).repeat_interleave(g, 0)
        vv_ = torch.from_numpy(vv[blk, pos % 16].astype(np.float64)).permute(1, 0, 2).repeat_interleave(g, 0)
        qq = torch.from_numpy(q[cu[i]:cu[i + 1]].astype(np.float64)).permute(1, 0, 2)  # [Hq, n, D]
        mask = torch.from_numpy(pos[None, :] <= (length - n + np.arange(n))[:, None])
        o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv_, attn_mask=mask, scale=w.scale)
        np.testing.assert_allclose(got[cu[i]:cu[i + 1]], o.permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_prefill_gqa_consistent_with_decode_and_closed_forms():
    qlens, lens = [7, 1, 20], [7, 50, 64]
    w, kv, vv, cu, q = _prefill_case("pfc", 8, 2, 64, 16, qlens, lens)
    got = paged.prefill_gqa(q, kv, vv, w.block_tables, w.context_lens, cu, w.scale)
    # the last new token of every sequence sees the whole context: decode over L
    last = q[cu[1:] - 1]
    dec = paged.decode_gqa(last, kv, vv, w.block_tables, w.context_lens, w.scale)
    np.testing.assert_allclose(got[cu[1:] - 1], dec, rtol=1e-12, atol=1e-13)
    # the first token of a prompt with no context attends only to itself: o = v_0 exactly
    v0 = vv[w.block_tables[0][0], 0]  # [Hkv, D]
    np.testing.assert_array_equal(got[0], np.repeat(v0, 4, axis=0))
    # a new token j of sequence 2 (context 44) equals decode over its first 44 + j + 1 positions
    j = 9
    dec_j = paged.decode_gqa(q[cu[2] + j][None], kv, vv, w.block_tables[2:3], np.array([44 + j + 1]), w.scale)
    np.testing.assert_allclose(got[cu[2] + j], dec_j[0], rtol=1e-12, atol=1e-13)


def test_prefill_gqa_sinks_consistent_with_decode():
    """With sinks, every new token equals the (independently pinned) decode with the
    same sinks over the positions it sees; -inf sinks change nothing."""
    qlens, lens = [7, 1, 20], [7, 50, 64]
    w, kv, vv, cu, q = _prefill_case("pfs", 8, 2, 64, 16, qlens, lens)
    sinks = np.array([-np.inf, 3.0, -1.0, 0.5, 8.0, -4.0, 1.5, 0.0])
    got = paged.prefill_gqa(q, kv, vv, w.block_tables, w.context_lens, cu, w.scale, sinks=sinks)
    for i in range(3):
        for j in range(qlens[i]):
            seen = lens[i] - qlens[i] + j + 1
            dec = paged.decode_gqa(q[cu[i] + j][None], kv, vv, w.block_tables[i:i + 1], np.array([seen]), w.scale,
                                   sinks=sinks)
            np.testing.assert_allclose(got[cu[i] + j], dec[0], rtol=1e-12, atol=1e-13)
    none = paged.prefill_gqa(q, kv, vv, w.block_tables, w.context_lens, cu, w.scale)
    np.testing.assert_array_equal(
        paged.prefill_gqa(q, kv, vv, w.block_tables, w.context_lens, cu, w.scale, sinks=np.full(8, -np.inf)), none)


# ---------------------------------------------------------------------------
# MLA latent cache: append / gather / block copy, and sinks in the MLA decode

def _mla_tables(lens, bs, num_blocks, seed):
    """Block tables dealing a seeded permutation of the pool's blocks to the sequences."""
    perm = np.random.default_rng(seed).permutation(num_blocks).astype(np.int32)
    width = max(-(-int(L) // bs) for L in lens)
    bt = np.full((len(lens), width), -1, np.int32)
    k = 0
    for i, L in enumerate(lens):
        n = -(-int(L) // bs)
        bt[i, :n] = perm[k:k + n]
        k += n
    return bt


def test_mla_append_gather_round_trip_and_untouched_blocks():
    nb, bs, r, p = 40, 16, 32, 8
    lens = np.array([1, 16, 17, 100, 63, 0, 200], np.int32)
    bt = _mla_tables(lens, bs, nb, 3)
    lat = np.full((nb, bs, r + p), 0xFFC1, np.uint16)  # a NaN pattern in every unwritten element
    before = lat.copy()
    slots = np.concatenate([bt[i][np.arange(L) // bs].astype(np.int64) * bs + np.arange(L) % bs
                            for i, L in enumerate(lens)])
    kvc = synth.normal_bf16(synth.stream_key("mlart", "c"), (len(slots), r))
    kpe = synth.normal_bf16(synth.stream_key("mlart", "p"), (len(slots), p))
    paged.append_mla(lat, kvc, kpe, slots)
    got = paged.gather_mla(lat, bt, lens)
    np.testing.assert_array_equal(got, np.concatenate([kvc, kpe], axis=1))
    used = set((slots // bs).tolist())
    free = [b for b in range(nb) if b not in used]
    np.testing.assert_array_equal(lat[free], before[free])
    assert paged.gather_mla(lat, bt[:0], lens[:0]).shape == (0, r + p)


def test_mla_append_and_gather_match_elementwise_loops():
    nb, bs, r, p = 5, 16, 16, 8
    lat = np.zeros((nb, bs, r + p), np.uint16)
    slots = np.array([17, -1, 3, 79, 40, 16], np.int64)
    kvc = synth.normal_bf16(synth.stream_key("mlaloop", "c"), (len(slots), r))
    kpe = synth.normal_bf16(synth.stream_key("mlaloop", "p"), (len(slots), p))
    paged.append_mla(lat, kvc, kpe, slots)
    expect = np.zeros_like(lat)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        b, o = divmod(int(s), bs)
        for e in range(r + p):
            expect[b, o, e] = kvc[t, e] if e < r else kpe[t, e - r]
    np.testing.assert_array_equal(lat, expect)
    bt = np.array([[1, 4, 0], [2, 0, 0]], np.int32)
    lens = np.array([35, 7], np.int32)
    got = paged.gather_mla(lat, bt, lens)
    row = 0
    for i in range(2):
        for t in range(int(lens[i])):
            for e in range(r + p):
                assert got[row, e] == lat[bt[i, t // bs], t % bs, e]
            row += 1
    assert row == got.shape[0]


def test_copy_blocks_is_copy_on_write():
    """After (src, dst) copies, a table that names dst where it named src gathers the
    same context (what a forked member's own table then reads), one source may feed
    several destinations, out-of-range pairs change nothing, and chained pairs are refused."""
    nb, bs, r, p = 12, 16, 16, 8
    lat = synth.random_u64(synth.stream_key("cow", "lat"), nb * bs * (r + p)).astype(np.uint16).reshape(nb, bs, r + p)
    ks = np.arange(nb * 2, dtype=np.float32).reshape(nb, 2)
    orig, orig_ks = lat.copy(), ks.copy()
    paged.copy_blocks([lat, ks], [(3, 9), (3, 10), (-1, 2), (4, nb)])
    for b in range(nb):
        src = 3 if b in (9, 10) else b
        np.testing.assert_array_equal(lat[b], orig[src])
        np.testing.assert_array_equal(ks[b], orig_ks[src])
    with pytest.raises(ValueError, match="independent"):
        paged.copy_blocks([lat], [(3, 9), (9, 10)])
    with pytest.raises(ValueError, match="independent"):
        paged.copy_blocks([lat], [(3, 9), (4, 9)])
    bt = np.array([[5, 3, 7]], np.int32)
    lens = np.array([40], np.int32)
    np.testing.assert_array_equal(paged.gather_mla(lat, np.array([[5, 9, 7]], np.int32), lens),
                                  paged.gather_mla(lat, bt, lens))


def mla_sink_case():
    """The reference's known answer as a shared-KV (MLA) decode with its sink.

    tests/test_deepseek_attention.py:100-118: query [0.5, -0.25], one key that is
    also the value [2, -1] (the shared-KV attention of attention.py:652-663 reads
    one latent row as key and value), scaling 0.5, a zero-logit zero-value sink,
    an ignored slot: output sigmoid(0.625) * [2, -1]. Here the latent row is
    c_kv = [2, -1, 0...], k_pe = 0; every slot past the one-token context holds NaN.
    """
    nb, bs, r, p = 2, 16, 16, 8
    lat = np.full((nb, bs, r + p), np.nan)
    lat[1, 0] = 0.0
    lat[1, 0, :2] = [2.0, -1.0]
    q = np.zeros((1, 1, r + p))
    q[0, 0, :2] = [0.5, -0.25]
    expected = np.zeros((1, 1, r))
    expected[0, 0, :2] = (1.0 / (1.0 + math.exp(-0.625))) * np.array([2.0, -1.0])
    return lat, q, np.array([[1]], np.int32), np.array([1], np.int32), 0.5, np.zeros(1), expected, r


def test_decode_mla_sink_reference_known_answer():
    lat, q, bt, lens, scale, sinks, expected, r = mla_sink_case()
    out = paged.decode_mla(q, lat, bt, lens, scale, kv_lora_rank=r, sinks=sinks)
    assert np.all(np.isfinite(out))
    np.testing.assert_allclose(out, expected, rtol=1e-12, atol=1e-12)


def test_decode_mla_sink_equals_a_zero_value_token():
    """Head h's sink s_h equals one more latent row with c_kv = 0 (a zero value) whose
    score against head h is exactly s_h. With every head's q_pe = a_h u (one shared
    direction u), the row k_pe = t u scores a_h t |u|^2 scale, so the sinks
    s_h = a_h t |u|^2 scale are matched for all heads by that single row."""
    rng = np.random.default_rng(11)
    b, h, r, p, bs, scale = 4, 6, 32, 8, 16, 0.1
    lens = np.array([0, 1, 30, 47], np.int32)
    nblk = (int(lens.max()) + 1 + bs - 1) // bs
    bt = np.arange(b * nblk, dtype=np.int32).reshape(b, nblk)
    lat = rng.standard_normal((b * nblk, bs, r + p))
    u = rng.standard_normal(p)
    a = rng.standard_normal(h)
    q = rng.standard_normal((b, h, r + p))
    q[:, :, r:] = a[None, :, None] * u[None, None, :]
    t = 1.7
    sinks = a * t * float(u @ u) * scale
    out = paged.decode_mla(q, lat, bt, lens, scale, kv_lora_rank=r, sinks=sinks)
    lat2 = lat.copy()
    for i in range(b):
        pos = int(lens[i])
        lat2[bt[i, pos // bs], pos % bs, :r] = 0.0
        lat2[bt[i, pos // bs], pos % bs, r:] = t * u
    ref = paged.decode_mla(q, lat2, bt, lens + 1, scale, kv_lora_rank=r)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    assert np.all(out[0] == 0.0)  # no context: the sink takes everything


def test_decode_mla_sink_closed_forms():
    """-inf sinks change nothing; n identical latent rows under a sink s give
    c_kv * n / (n + e^(s - c)), c the common score."""
    rng = np.random.default_rng(12)
    b, h, r, p, bs, scale = 3, 4, 16, 8, 16, 0.25
    lens = np.array([5, 16, 31], np.int32)
    bt = np.arange(b * 2, dtype=np.int32).reshape(b, 2)
    lat = rng.standard_normal((b * 2, bs, r + p))
    q = rng.standard_normal((b, h, r + p))
    none = paged.decode_mla(q, lat, bt, lens, scale, kv_lora_rank=r)
    np.testing.assert_array_equal(paged.decode_mla(q, lat, bt, lens, scale, kv_lora_rank=r,
                                                   sinks=np.full(h, -np.inf)), none)
    lat[:] = lat[0, 0]
    sinks = np.array([-1.0, 0.0, 2.0, 5.0])
    out = paged.decode_mla(q, lat, bt, lens, scale, kv_lora_rank=r, sinks=sinks)
    for i in range(b):
        for hh in range(h):
            c = float(q[i, hh] @ lat[0, 0]) * scale
            n = float(lens[i])
            np.testing.assert_allclose(out[i, hh], lat[0, 0, :r] * n / (n + math.exp(sinks[hh] - c)), rtol=1e-12)
