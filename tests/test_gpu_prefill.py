"""GPU parity of varlen (chunked) prefill against the float64 oracle.

Each case mixes sequences that prefill a whole prompt, prefill a chunk after
cached context (an earlier chunk or a prefix-cache hit), bring a single token,
or bring none. The cached context is written through the oracle's append and
uploaded; prefill_gqa then appends the new tokens itself (compared bit-exact
with the oracle's append) and attends causally (tolerance as for decode:
|got - ref| <= 2e-2 + 1e-2 |ref|, relative L2 <= 1e-2). Unowned bf16 slots
hold NaN.
"""

import math

import numpy as np
import pytest
import torch

from kvcase import bits_of, check_attention, slots_for, to_dev_bits
from oracle import fp8, paged
from wavelet_amd import PagedKVCache, paged_decode_gqa, prefill_gqa, synth

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _case(cuda, name, hq, hkv, d, bs, qlens, lens, kv_dtype):
    qlens, lens = np.asarray(qlens), np.asarray(lens)
    w = synth.make_decode_workload(name, batch=len(lens), num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=bs, context_lens=lens)
    is_fp8 = kv_dtype == "fp8_e4m3"
    NB = w.num_blocks
    # cached context: positions [0, L - n) of every sequence, written by the oracle
    ctx = lens - qlens
    cslots = slots_for(w, np.zeros(w.batch, np.int64), ctx)
    kb = synth.normal_bf16(synth.stream_key(name, "ck"), (len(cslots), hkv, d))
    vb = synth.normal_bf16(synth.stream_key(name, "cv"), (len(cslots), hkv, d))
    if is_fp8:
        kc, vc = paged.empty_cache(NB, bs, hkv, d, dtype=np.uint8)
        ks = np.zeros((NB, hkv), np.float32)
        vs = np.zeros((NB, hkv), np.float32)
        paged.append_fp8(kc, vc, ks, vs, kb, vb, cslots)
    else:
        kc, vc = paged.empty_cache(NB, bs, hkv, d, dtype=np.uint16, fill=0x7FC0)
        ks = vs = None
        paged.append_bf16(kc, vc, kb, vb, cslots)
    cache = PagedKVCache(NB, bs, hkv, d, kv_dtype=kv_dtype, device=cuda)
    dt = torch.uint8 if is_fp8 else BF16
    cache.k.copy_(to_dev_bits(kc, dt, cuda).view(cache.k.dtype))
    cache.v.copy_(to_dev_bits(vc, dt, cuda).view(cache.v.dtype))
    if is_fp8:
        cache.k_scale.copy_(torch.from_numpy(ks).to(cuda))
        cache.v_scale.copy_(torch.from_numpy(vs).to(cuda))
    # the new tokens: positions [L - n, L)
    nslots = slots_for(w, ctx, lens)
    T = int(qlens.sum())
    assert len(nslots) == T
    kn = synth.normal_bf16(synth.stream_key(name, "nk"), (T, hkv, d))
    vn = synth.normal_bf16(synth.stream_key(name, "nv"), (T, hkv, d))
    q = synth.normal_bf16(synth.stream_key(name, "q"), (T, hq, d))
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    return w, cache, (kc, vc, ks, vs), (kn, vn, q, nslots, cu)


def _run_and_check(cuda, w, cache, host, new, what, sinks=None):
    kc, vc, ks, vs = host
    kn, vn, q, nslots, cu = new
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    out = prefill_gqa(to_dev_bits(q, BF16, cuda), cache, bt, sl, torch.from_numpy(cu).to(cuda), w.scale,
                      key=to_dev_bits(kn, BF16, cuda), value=to_dev_bits(vn, BF16, cuda),
                      slot_mapping=torch.from_numpy(nslots).to(cuda),
                      sinks=None if sinks is None else torch.from_numpy(sinks).to(cuda))
    if ks is not None:
        paged.append_fp8(kc, vc, ks, vs, kn, vn, nslots)
        kf = fp8.dequantize(paged.k_logical(kc).reshape(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim),
                            ks[:, None, :, None])
        vf = fp8.dequantize(paged.v_logical(vc), vs[:, None, :, None])
    else:
        paged.append_bf16(kc, vc, kn, vn, nslots)
        kl, vl = paged.logical_kv(kc, vc)
        kf, vf = paged.bf16_to_f32(kl), paged.bf16_to_f32(vl)
    assert np.array_equal(bits_of(cache.k), kc) and np.array_equal(bits_of(cache.v), vc), f"{what}: cache"
    if ks is not None:
        np.testing.assert_array_equal(cache.k_scale.cpu().numpy(), ks)
        np.testing.assert_array_equal(cache.v_scale.cpu().numpy(), vs)
    ref = paged.prefill_gqa(paged.bf16_to_f32(q), kf, vf, w.block_tables, w.context_lens, cu, w.scale, sinks=sinks)
    if sinks is not None:
        plain = paged.prefill_gqa(paged.bf16_to_f32(q), kf, vf, w.block_tables, w.context_lens, cu, w.scale)
        assert np.abs(ref - plain).max() > 0.1, f"{what}: the sinks must matter in this case"
    a, r = check_attention(paged.bf16_to_f32(bits_of(out)), ref, what)
    print(f"{what}: err abs {a:.2e} rel {r:.2e}")
    return out


# (new tokens, total length) per sequence: whole prompts, chunks after context, one token, none
MIX = ([37, 16, 1, 130, 0, 64, 200], [37, 300, 50, 1000, 20, 64, 900])


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
@pytest.mark.parametrize("hq,hkv,d,bs", [(32, 8, 128, 16), (14, 2, 64, 16), (28, 4, 128, 16), (16, 16, 128, 64),
                                         (8, 1, 64, 32), (16, 4, 128, 128), (8, 2, 64, 256), (16, 8, 128, 16)])
def test_prefill_varlen_chunked(cuda, kv_dtype, hq, hkv, d, bs):
    name = f"pf{kv_dtype}{hq}{hkv}{d}{bs}"
    w, cache, host, new = _case(cuda, name, hq, hkv, d, bs, *MIX, kv_dtype)
    _run_and_check(cuda, w, cache, host, new, name)


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
@pytest.mark.parametrize("hq,hkv,d,bs", [(32, 8, 128, 16), (14, 2, 64, 16)])
def test_prefill_with_attention_sinks(cuda, kv_dtype, hq, hkv, d, bs):
    """Per-head sinks (a zero-value logit, wavelet/trainer/models/deepseek_v4/attention.py:89-95):
    none (-inf), dominant, strongly negative and moderate ones, on the mixed varlen case."""
    name = f"pfsink{kv_dtype}{hq}{hkv}{d}{bs}"
    w, cache, host, new = _case(cuda, name, hq, hkv, d, bs, *MIX, kv_dtype)
    sinks = (synth.normal(synth.stream_key(name, "sinks"), hq) * 2.0).astype(np.float32)
    sinks[0], sinks[1], sinks[2] = -np.inf, 9.0, -6.0
    _run_and_check(cuda, w, cache, host, new, name, sinks=sinks)


def test_prefill_long_prompt_and_long_context_chunk(cuda):
    """A 2,000-token prompt (ranges of 64 blocks, many query tiles) and a 100-token chunk after 3,000."""
    w, cache, host, new = _case(cuda, "pflong", 32, 8, 128, 16, [2000, 100], [2000, 3100], "bf16")
    _run_and_check(cuda, w, cache, host, new, "long")


def test_prefill_single_tokens_equal_decode(cuda):
    """One new token per sequence is a decode step: prefill and the decode kernel agree."""
    qlens, lens = [1] * 6, [1, 17, 64, 300, 1024, 2049]
    w, cache, host, new = _case(cuda, "pfdec", 28, 4, 128, 16, qlens, lens, "bf16")
    out = _run_and_check(cuda, w, cache, host, new, "single tokens")
    q = new[2]
    dec = paged_decode_gqa(to_dev_bits(q, BF16, cuda), cache, torch.from_numpy(w.block_tables).to(cuda),
                           torch.from_numpy(w.context_lens).to(cuda), w.scale)
    torch.testing.assert_close(out.float(), dec.float(), atol=2e-2, rtol=1e-2)
