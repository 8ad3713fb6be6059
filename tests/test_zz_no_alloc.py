"""The allocation-free fused decode (wkv_append_paged_decode_gqa_noalloc) against the
workspace entry point (wkv_append_paged_decode_gqa), through the C ABI.

Two calls in a row on one GPU, the second with a smaller batch and shorter
contexts (the static scratch then still holds the first call's partials),
each on a geometry whose contexts span several workgroup chunks so the
split-K partials and the merge kernel are in play. The outputs and the caches
after the fused append must be bit-identical to the workspace path's (the
same kernels, the same partial layout). A geometry needing more scratch than
the static array holds is refused before any launch.
"""

import ctypes

import numpy as np
import pytest
import torch

from kvcase import bits_of
from wavelet_amd import PagedKVCache, _lib, decode_plan, synth

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _case(cuda, name, lens, hq, hkv, d, kv_dtype, partition):
    w = synth.make_decode_workload(name, batch=len(lens), num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=16, context_lens=np.asarray(lens))
    gen = torch.Generator(device=cuda)
    gen.manual_seed(len(lens) * 1000 + hq)
    caches = [PagedKVCache(w.num_blocks, 16, hkv, d, kv_dtype=kv_dtype, device=cuda) for _ in range(2)]
    if kv_dtype == "bf16":
        caches[0].k.normal_(generator=gen)
        caches[0].v.normal_(generator=gen)
    else:
        for t in (caches[0].k, caches[0].v):
            t.copy_(torch.randint(0, 256, t.shape, generator=gen, device=cuda, dtype=torch.int32).to(torch.uint8)
                    & 0xF7)
        caches[0].k_scale.fill_(2.0 ** -8)
        caches[0].v_scale.fill_(2.0 ** -8)
    for name_ in ("k", "v", "k_scale", "v_scale"):
        a, b = getattr(caches[0], name_), getattr(caches[1], name_)
        if a is not None:
            b.copy_(a)
    B = w.batch
    q = torch.randn((B, hq, d), generator=gen, device=cuda).to(BF16)
    key = torch.randn((B, hkv, d), generator=gen, device=cuda).to(BF16)
    val = torch.randn((B, hkv, d), generator=gen, device=cuda).to(BF16)
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    slots = torch.from_numpy(w.new_token_slots()).to(cuda)
    max_seq = int(w.context_lens.max())
    _, _, chunks = decode_plan(B, hkv, max_seq, 16, partition)
    assert chunks > 1, f"{name}: the geometry must leave split-K partials"
    lib = _lib.load()
    stream = torch.cuda.current_stream(cuda).cuda_stream
    need = lib.wkv_decode_workspace_size(B, hq, d, max_seq, partition)
    ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device=cuda)
    outs = [torch.full((B, hq, d), float("nan"), dtype=BF16, device=cuda) for _ in range(2)]
    head = lambda c: (ctypes.byref(c.descriptor()), key.data_ptr(), key.stride(0), key.stride(1),  # noqa: E731
                      val.data_ptr(), val.stride(0), val.stride(1), slots.data_ptr())
    tail = lambda o: (q.data_ptr(), q.stride(0), q.stride(1), o.data_ptr(), hq, bt.data_ptr(),  # noqa: E731
                      bt.stride(0), bt.shape[1], sl.data_ptr(), B, max_seq, ctypes.c_float(w.scale), partition)
    torch.cuda.synchronize()
    print(f"noalloc case {name}: B={B} {hq}/{hkv} d={d} {kv_dtype} P={partition} chunks={chunks}", flush=True)
    rc = lib.wkv_append_paged_decode_gqa(*head(caches[0]), *tail(outs[0]), ws.data_ptr(), ws.numel(), None, stream)
    _lib.check(rc, "workspace path")
    rc = lib.wkv_append_paged_decode_gqa_noalloc(*head(caches[1]), *tail(outs[1]), None, stream)
    _lib.check(rc, "allocation-free path")
    torch.cuda.synchronize()
    assert np.array_equal(bits_of(outs[0]), bits_of(outs[1])), f"{name}: outputs differ"
    assert bool(torch.isfinite(outs[1].float()).all()), f"{name}: non-finite output"
    for name_ in ("k", "v", "k_scale", "v_scale"):
        a, b = getattr(caches[0], name_), getattr(caches[1], name_)
        if a is not None:
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"{name}: cache {name_} differs"


@pytest.mark.parametrize("kv_dtype,hq,hkv,d", [("bf16", 32, 8, 128), ("fp8_e4m3", 14, 2, 64)])
def test_noalloc_matches_workspace_path_on_two_calls(cuda, kv_dtype, hq, hkv, d):
    lens1 = [8192, 1, 17, 1500, 4096, 6000, 333, 8000, 2048, 7777, 64, 5000]
    _case(cuda, f"noalloc1{kv_dtype}", lens1, hq, hkv, d, kv_dtype, 128)
    lens2 = [3000, 2, 1024, 700, 2500]  # smaller batch, shorter contexts: fewer partial slots than call 1
    _case(cuda, f"noalloc2{kv_dtype}", lens2, hq, hkv, d, kv_dtype, 128)


def test_noalloc_refuses_geometries_beyond_its_scratch(cuda):
    """4,096 sequences x 32 heads at 64 chunks of partials need ~4.4 GB: refused on the host, no launch."""
    lib = _lib.load()
    cache = PagedKVCache(64, 16, 8, 128, device=cuda)
    B, hq, max_seq = 4096, 32, 65536
    need = lib.wkv_decode_workspace_size(B, hq, 128, max_seq, 1024)
    assert need > _lib.WKV_NOALLOC_SCRATCH_BYTES
    buf = torch.zeros(1024, dtype=torch.int64, device=cuda)  # stands in for every pointer argument
    p = buf.data_ptr()
    rc = lib.wkv_append_paged_decode_gqa_noalloc(
        ctypes.byref(cache.descriptor()), p, 8 * 128, 128, p, 8 * 128, 128, p, p, hq * 128, 128, p, hq, p, 4096, 4096,
        p, B, max_seq, ctypes.c_float(0.1), 128, None, torch.cuda.current_stream(cuda).cuda_stream)
    assert rc == _lib.WKV_ERR_INVALID
    msg = _lib.last_error()
    assert "static scratch" in msg and str(need) in msg, msg
