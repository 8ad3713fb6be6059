"""GPU parity of the attention-sink decode (wkv_paged_decode_gqa_sinks and
wkv_append_paged_decode_gqa_sinks) against the float64 oracle.

A sink is one more logit per query head whose value vector is zero
(wavelet/trainer/models/deepseek_v4/attention.py:89-95). Tolerance as for
the plain decode (kvcase.check_attention: max |err| <= 2e-2 outright,
|err| <= 2e-2 + 1e-2 |ref| elementwise, relative L2 <= 1e-2). Slots outside
every context hold NaN. The partitions cover the three places a sink enters
the denominator: a one-wave chunk, the in-workgroup merge of several waves,
and the split-K merge kernel.
"""

import numpy as np
import pytest
import torch

from kvcase import bits_of, check_attention, slots_for, to_dev_bits
from oracle import paged
from test_gpu_decode import _bf16_caches, _to_physical
from wavelet_amd import PagedKVCache, decode_plan, paged_decode_gqa, synth

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _sinks(hq: int, tag: str) -> np.ndarray:
    """Per-head sinks spanning 'no sink' to 'sink dominates': -inf, large
    positive, moderate values of both signs."""
    s = synth.normal(synth.stream_key("sinks", tag), hq).astype(np.float32) * 2.0
    s[0] = -np.inf
    if hq > 1:
        s[1] = 9.0
    if hq > 2:
        s[2] = -6.0
    return s


def _cache(w, cuda, k_log, v_log):
    cache = PagedKVCache(w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, device=cuda)
    kp, vp = _to_physical(k_log, v_log)
    cache.k.copy_(to_dev_bits(kp, BF16, cuda))
    cache.v.copy_(to_dev_bits(vp, BF16, cuda))
    return cache


def test_decode_sinks_reference_known_answer(cuda):
    """The reference's sigmoid(0.625) * [2, -1] with its zero-logit sink passed as a sink."""
    from test_oracle import sink_case

    kc, vc, q, bt, lens, scale, sinks, expected = sink_case()
    w = synth.DecodeWorkload("sink", num_blocks=2, block_size=16, num_kv_heads=1, num_q_heads=1, head_dim=64,
                             context_lens=lens.astype(np.int32), block_tables=bt, scale=scale)
    cache = _cache(w, cuda, paged.f32_to_bf16(kc), paged.f32_to_bf16(vc))
    out = paged_decode_gqa(to_dev_bits(paged.f32_to_bf16(q), BF16, cuda), cache, torch.from_numpy(bt).to(cuda),
                           torch.from_numpy(lens).to(cuda), scale, sinks=torch.from_numpy(sinks).to(cuda))
    got = paged.bf16_to_f32(bits_of(out))
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, expected, atol=1e-2, rtol=0)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (8, 8, 64)])
def test_decode_sinks_match_oracle(cuda, hq, hkv, d):
    shapes = set()
    # long contexts: several waves per workgroup and split-K chunks; short ones fit one wave
    for lens, parts in ((np.array([0, 1, 17, 256, 257, 700, 1024, 3000]), (16, 64, 256, 0)),
                        (np.array([0, 1, 15, 16, 100, 255]), (256, 0))):
        w = synth.make_decode_workload(f"sinks{hq}x{hkv}x{d}L{int(lens.max())}", batch=len(lens), num_kv_heads=hkv,
                                       num_q_heads=hq, head_dim=d, block_size=16, context_lens=lens)
        k, v = _bf16_caches(w, "s")
        q = synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, hq, d))
        sinks = _sinks(hq, w.name)
        cache = _cache(w, cuda, k, v)
        qd, sd = to_dev_bits(q, BF16, cuda), torch.from_numpy(sinks).to(cuda)
        bt, sl = torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda)
        qf, kf, vf = paged.bf16_to_f32(q), paged.bf16_to_f32(k), paged.bf16_to_f32(v)
        ref = paged.decode_gqa(qf, kf, vf, w.block_tables, w.context_lens, w.scale, sinks=sinks)
        plain = paged.decode_gqa(qf, kf, vf, w.block_tables, w.context_lens, w.scale)
        assert np.abs(ref - plain).max() > 0.1, "the sinks must matter in this case"
        for p in parts:
            shapes.add(decode_plan(w.batch, hkv, int(lens.max()), w.block_size, p)[1:])
            out = paged_decode_gqa(qd, cache, bt, sl, w.scale, partition_size=p, sinks=sd)
            got = paged.bf16_to_f32(bits_of(out))
            a, r = check_attention(got, ref, f"{w.name} sinks P={p}")
            print(f"{w.name} sinks P={p}: err abs {a:.2e} rel {r:.2e}")
    waves = {wv for wv, _ in shapes}
    chunks = {c for _, c in shapes}
    assert 1 in waves and max(waves) > 1 and max(chunks) > 1, shapes  # all three sink sites ran


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp8_e4m3"])
def test_fused_append_decode_sinks_equals_append_then_decode(cuda, kv_dtype):
    """The fused step with sinks leaves the cache as the append does and attends as the separate
    decode with the same sinks (bf16: within tolerance; fp8: bit-identical, as without sinks)."""
    hq, hkv, d, bs = 16, 4, 128, 16
    lens = np.array([1, 2, 17, 300, 1025])
    w = synth.make_decode_workload(f"fsinks{kv_dtype}", batch=len(lens), num_kv_heads=hkv, num_q_heads=hq,
                                   head_dim=d, block_size=bs, context_lens=lens)
    caches = [PagedKVCache(w.num_blocks, bs, hkv, d, kv_dtype=kv_dtype, device=cuda) for _ in range(2)]
    ctx = w.context_lens.astype(np.int64)
    pslots = slots_for(w, np.zeros(w.batch, np.int64), ctx - 1)
    kp = synth.normal_bf16(synth.stream_key(w.name, "pk"), (len(pslots), hkv, d))
    vp = synth.normal_bf16(synth.stream_key(w.name, "pv"), (len(pslots), hkv, d))
    for c in caches:
        c.append(to_dev_bits(kp, BF16, cuda), to_dev_bits(vp, BF16, cuda), torch.from_numpy(pslots).to(cuda))
    nslots = torch.from_numpy(w.new_token_slots()).to(cuda)
    kn = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "nk"), (w.batch, hkv, d)), BF16, cuda)
    vn = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "nv"), (w.batch, hkv, d)), BF16, cuda)
    q = to_dev_bits(synth.normal_bf16(synth.stream_key(w.name, "q"), (w.batch, hq, d)), BF16, cuda)
    sd = torch.from_numpy(_sinks(hq, w.name)).to(cuda)
    bt, sl = torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda)
    caches[0].append(kn, vn, nslots)
    for p in (0, 4 * bs):
        ref_out = paged_decode_gqa(q, caches[0], bt, sl, w.scale, partition_size=p, sinks=sd)
        out = paged_decode_gqa(q, caches[1], bt, sl, w.scale, partition_size=p, new_key=kn, new_value=vn,
                               slot_mapping=nslots, sinks=sd)
        torch.cuda.synchronize()
        assert torch.equal(caches[0].k.view(torch.uint8), caches[1].k.view(torch.uint8)), f"K differs (P={p})"
        assert torch.equal(caches[0].v.view(torch.uint8), caches[1].v.view(torch.uint8)), f"V differs (P={p})"
        if kv_dtype == "fp8_e4m3":
            assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), f"output differs (P={p})"
        else:
            torch.testing.assert_close(out.float(), ref_out.float(), atol=2e-2, rtol=1e-2,
                                       msg=lambda m: f"fused vs separate (P={p}): {m}")


def test_decode_sinks_rejects_bad_tensors(cuda):
    w = synth.make_decode_workload("sinkbad", batch=2, num_kv_heads=2, num_q_heads=4, head_dim=64, block_size=16,
                                   context_lens=np.array([3, 5]))
    cache = PagedKVCache(w.num_blocks, 16, 2, 64, device=cuda)
    q = torch.zeros((2, 4, 64), dtype=BF16, device=cuda)
    bt, sl = torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda)
    for bad in (torch.zeros(3, device=cuda), torch.zeros(4, dtype=torch.float64, device=cuda), torch.zeros(4)):
        with pytest.raises(ValueError):
            paged_decode_gqa(q, cache, bt, sl, w.scale, sinks=bad)
