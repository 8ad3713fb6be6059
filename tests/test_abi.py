"""The C ABI on a host without a GPU: the library loads, exports every symbol
include/wkv.h declares, and rejects bad arguments before any launch."""

import ctypes
import re
from pathlib import Path

import pytest

from wavelet_amd import _lib


def _no_gpu() -> bool:
    try:
        import torch

        return not torch.cuda.is_available()
    except Exception:
        return True


# These tests hand the library fake device pointers and rely on host-side
# validation rejecting every call before a launch; they run only where no GPU
# is visible, so a validation regression can never reach a real device.
host_only = pytest.mark.skipif(not _no_gpu(), reason="fake device pointers: host-only test")

HEADER = Path(__file__).resolve().parents[1] / "include" / "wkv.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(wkv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 11
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"libwkv.so lacks {missing}"
    # and the ctypes table covers the whole header
    assert sorted(_lib._SIGNATURES) == names


def test_version():
    assert _lib.load().wkv_version() == 1


def _desc(**kw):
    base = dict(k=16, v=32, k_scale=None, v_scale=None, num_blocks=4, block_size=16, num_kv_heads=2,
                head_dim=128, kv_dtype=_lib.WKV_KV_BF16)
    base.update(kw)
    return _lib.WkvCache(**base)


@host_only
def test_append_rejects_bad_arguments_before_launch():
    lib = _lib.load()
    # NULL descriptor
    assert lib.wkv_append(None, None, 0, 0, None, 0, 0, None, 1, None) == _lib.WKV_ERR_INVALID
    assert "NULL" in _lib.last_error()
    # misaligned cache pointer
    d = _desc(k=17)
    assert lib.wkv_append(ctypes.byref(d), 16, 1024, 128, 16, 1024, 128, 16, 1, None) == _lib.WKV_ERR_INVALID
    # unsupported head_dim
    d = _desc(head_dim=96)
    assert lib.wkv_append(ctypes.byref(d), 16, 1024, 128, 16, 1024, 128, 16, 1, None) == _lib.WKV_ERR_UNSUPPORTED
    # block_size not a multiple of 16
    d = _desc(block_size=24)
    assert lib.wkv_append(ctypes.byref(d), 16, 1024, 128, 16, 1024, 128, 16, 1, None) == _lib.WKV_ERR_INVALID
    # bf16 entry point on an fp8 cache
    d = _desc(kv_dtype=_lib.WKV_KV_FP8_E4M3, k_scale=48, v_scale=64)
    assert lib.wkv_append(ctypes.byref(d), 16, 1024, 128, 16, 1024, 128, 16, 1, None) == _lib.WKV_ERR_INVALID
    # fp8 cache without scales
    d = _desc(kv_dtype=_lib.WKV_KV_FP8_E4M3)
    assert lib.wkv_append_fp8(ctypes.byref(d), 16, 1024, 128, 16, 1024, 128, 16, 1, None) == _lib.WKV_ERR_INVALID
    # key stride not a multiple of 8
    d = _desc()
    assert lib.wkv_append(ctypes.byref(d), 16, 1023, 128, 16, 1024, 128, 16, 1, None) == _lib.WKV_ERR_INVALID
    assert "strides" in _lib.last_error()
    # zero tokens is a no-op success
    assert lib.wkv_append(ctypes.byref(d), None, 0, 0, None, 0, 0, None, 0, None) == _lib.WKV_OK


@host_only
def test_decode_rejects_bad_arguments_before_launch():
    lib = _lib.load()
    d = _desc()
    f = lib.wkv_paged_decode_gqa
    # Hq not a multiple of Hkv
    assert f(ctypes.byref(d), 16, 1024, 128, 16, 3, 16, 4, 4, 16, 1, 64, 0.1, 0, None, 0, None, None) == _lib.WKV_ERR_INVALID
    # group size 32 > 16 is not supported
    assert f(ctypes.byref(d), 16, 8192, 128, 16, 64, 16, 4, 4, 16, 1, 64, 0.1, 0, None, 0, None, None) == _lib.WKV_ERR_UNSUPPORTED
    # partition not a multiple of 16
    assert f(ctypes.byref(d), 16, 1024, 128, 16, 8, 16, 4, 4, 16, 1, 64, 0.1, 24, None, 0, None, None) == _lib.WKV_ERR_INVALID
    # workspace missing when the context spans several workgroups (64 partitions of 16)
    assert f(ctypes.byref(d), 16, 1024, 128, 16, 8, 16, 64, 64, 16, 1, 1024, 0.1, 16, None, 0, None, None) == _lib.WKV_ERR_INVALID
    assert "workspace" in _lib.last_error()
    # a partition spanning more than 64 blocks
    assert f(ctypes.byref(d), 16, 1024, 128, 16, 8, 16, 4, 4, 16, 1, 64, 0.1, 2048, None, 0, None, None) == _lib.WKV_ERR_INVALID
    # fused append: partition must be a multiple of the block size
    g = lib.wkv_append_paged_decode_gqa
    assert g(ctypes.byref(d), 16, 256, 128, 16, 256, 128, 16, 16, 1024, 128, 16, 8, 16, 4, 4, 16, 1, 64, 0.1, 24,
             None, 0, None, None) == _lib.WKV_ERR_INVALID
    assert g(ctypes.byref(d), None, 256, 128, 16, 256, 128, 16, 16, 1024, 128, 16, 8, 16, 4, 4, 16, 1, 64, 0.1, 0,
             None, 0, None, None) == _lib.WKV_ERR_INVALID
    # non-finite scale
    assert f(ctypes.byref(d), 16, 1024, 128, 16, 8, 16, 4, 4, 16, 1, 64, float("nan"), 0, None, 0, None, None) == _lib.WKV_ERR_INVALID
    # empty batch is a no-op success
    assert f(ctypes.byref(d), 16, 1024, 128, 16, 8, 16, 4, 4, 16, 0, 64, 0.1, 0, None, 0, None, None) == _lib.WKV_OK
    # dispatch order: batch range and NULL pointers checked before any launch; empty batch is a no-op
    o = lib.wkv_decode_order
    assert o(16, -1, 16, None) == _lib.WKV_ERR_INVALID
    assert o(16, 65536, 16, None) == _lib.WKV_ERR_INVALID
    assert o(None, 4, 16, None) == _lib.WKV_ERR_INVALID
    assert o(16, 4, None, None) == _lib.WKV_ERR_INVALID
    assert o(None, 0, None, None) == _lib.WKV_OK
    # the group-aware order: the same checks plus the group and the decode geometry
    go = lib.wkv_grouped_decode_order
    assert go(16, 8, 0, 4, 4096, 16, 0, 16, None) == _lib.WKV_ERR_INVALID  # group_size 0
    assert go(16, 8, 9, 4, 4096, 16, 0, 16, None) == _lib.WKV_ERR_INVALID  # group larger than the batch
    assert go(16, 8, 4, 0, 4096, 16, 0, 16, None) == _lib.WKV_ERR_INVALID  # no KV heads
    assert go(16, 8, 4, 4, 4096, 24, 0, 16, None) == _lib.WKV_ERR_INVALID  # block size not a multiple of 16
    assert go(None, 8, 4, 4, 4096, 16, 0, 16, None) == _lib.WKV_ERR_INVALID
    assert go(16, 8, 4, 4, 4096, 16, 0, None, None) == _lib.WKV_ERR_INVALID
    assert go(None, 0, 0, 0, 0, 0, 0, None, None) == _lib.WKV_OK  # empty batch: a no-op


@host_only
def test_mla_rejects_unsupported_geometry():
    lib = _lib.load()
    m = _lib.WkvMlaCache(latent=16, num_blocks=4, block_size=64, kv_lora_rank=256, rope_dim=64)
    rc = lib.wkv_paged_decode_mla(ctypes.byref(m), 16, 0, 0, 16, 0, 0, 16, 128, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0, None)
    assert rc == _lib.WKV_ERR_UNSUPPORTED
    m = _lib.WkvMlaCache(latent=16, num_blocks=4, block_size=64, kv_lora_rank=512, rope_dim=64)
    rc = lib.wkv_paged_decode_mla(ctypes.byref(m), 16, 0, 0, 16, 0, 0, 16, 48, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0, None)
    assert rc == _lib.WKV_ERR_UNSUPPORTED
    # fused append + decode: inputs checked before any launch
    g = lib.wkv_append_paged_decode_mla
    assert g(ctypes.byref(m), None, 512, 16, 64, 16, 16, 0, 0, 16, 0, 0, 16, 128, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0,
             None) == _lib.WKV_ERR_INVALID
    assert g(ctypes.byref(m), 16, 511, 16, 64, 16, 16, 0, 0, 16, 0, 0, 16, 128, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0,
             None) == _lib.WKV_ERR_INVALID
    assert g(ctypes.byref(m), 16, 512, 16, 64, None, 16, 0, 0, 16, 0, 0, 16, 128, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0,
             None) == _lib.WKV_ERR_INVALID


def test_workspace_sizes():
    lib = _lib.load()
    # 64 seqs x 32 heads x ceil(4096/256)=16 partitions x (128 + 2) floats
    assert lib.wkv_decode_workspace_size(64, 32, 128, 4096, 256) == 64 * 32 * 16 * 130 * 4
    assert lib.wkv_decode_workspace_size(64, 32, 128, 4096, 0) == 64 * 32 * 32 * 130 * 4
    assert lib.wkv_decode_workspace_size(-1, 32, 128, 4096, 0) == -1
    # MLA: 32 seqs x 128 heads x 8 partitions x (bf16 partial of 512 + fp32 maximum and sum)
    assert lib.wkv_mla_workspace_size(32, 128, 512, 4096, 512) == 32 * 128 * 8 * (512 * 2 + 8)


@host_only
def test_status_codes_map_to_python_exceptions():
    lib = _lib.load()
    lib.wkv_append(None, None, 0, 0, None, 0, 0, None, 1, None)
    with pytest.raises(ValueError, match="NULL"):
        _lib.check(_lib.WKV_ERR_INVALID, "append")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.WKV_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.WKV_ERR_LAUNCH, "x")


def test_decode_plan_shapes_and_errors():
    """The launch shape is host logic: an eighth of the longest context per wave (8-wave workgroups),
    fewer tokens when the batch is too small to fill the GPU, never below 128 tokens or above 64 blocks."""
    from wavelet_amd import decode_plan

    assert decode_plan(64, 8, 4096, 16) == (512, 8, 1)  # Qwen3-4B headline
    assert decode_plan(64, 8, 8192, 16) == (1024, 8, 1)  # var-length, longest 8,192
    assert decode_plan(128, 2, 2048, 16) == (256, 8, 1)  # Qwen2.5-0.5B
    assert decode_plan(1, 8, 4096, 16) == (128, 8, 4)  # one sequence: more, shorter partitions
    assert decode_plan(64, 8, 65536, 16) == (1024, 8, 8)  # long context: 1,024-token partitions, merged
    assert decode_plan(64, 8, 4096, 16, 1024) == (1024, 4, 1)  # the caller's partition wins
    assert decode_plan(64, 8, 100, 16) == (128, 1, 1)
    assert decode_plan(64, 8, 4096, 64) == (512, 8, 1)
    lib = _lib.load()
    o = ctypes.c_int32()
    assert lib.wkv_decode_plan(64, 8, 4096, 8, 0, ctypes.byref(o), ctypes.byref(o), ctypes.byref(o)) == _lib.WKV_ERR_INVALID
    assert lib.wkv_decode_plan(64, 0, 4096, 16, 0, ctypes.byref(o), ctypes.byref(o), ctypes.byref(o)) == _lib.WKV_ERR_INVALID
    assert lib.wkv_decode_plan(64, 8, 4096, 16, 0, None, ctypes.byref(o), ctypes.byref(o)) == _lib.WKV_ERR_INVALID


@host_only
def test_prefill_rejects_bad_arguments_before_launch():
    lib = _lib.load()
    d = _desc()  # 2 KV heads, d=128, blocks of 16
    base = dict(key=None, kst=0, ksh=0, value=None, vst=0, vsh=0, slots=None, ntok=0, q=16, qst=1024, qsh=128,
                out=16, ost=1024, osh=128, hq=8, cu=16, sl=16, bt=16, bts=4, mb=4, batch=1, mq=16, ms=64, scale=0.1)

    def call(**kw):
        a = dict(base, **kw)
        return lib.wkv_prefill_gqa(ctypes.byref(d), a["key"], a["kst"], a["ksh"], a["value"], a["vst"], a["vsh"],
                                   a["slots"], a["ntok"], a["q"], a["qst"], a["qsh"], a["out"], a["ost"], a["osh"],
                                   a["hq"], a["cu"], a["sl"], a["bt"], a["bts"], a["mb"], a["batch"], a["mq"],
                                   a["ms"], a["scale"], None)

    assert call(hq=3) == _lib.WKV_ERR_INVALID  # not a multiple of the KV heads
    assert call(q=17) == _lib.WKV_ERR_INVALID
    assert "aligned" in _lib.last_error()
    assert call(qst=1020) == _lib.WKV_ERR_INVALID  # q strides: multiples of 8
    assert call(out=None) == _lib.WKV_ERR_INVALID
    assert call(osh=2) == _lib.WKV_ERR_INVALID  # out strides: multiples of 4
    assert call(cu=None) == _lib.WKV_ERR_INVALID
    assert call(bts=2) == _lib.WKV_ERR_INVALID  # table stride below its width
    assert call(scale=float("inf")) == _lib.WKV_ERR_INVALID
    assert call(batch=70000) == _lib.WKV_ERR_INVALID
    assert call(ntok=-1) == _lib.WKV_ERR_INVALID
    # the append half: a key without a value is rejected before anything runs
    assert call(key=16, kst=256, ksh=128, slots=16, ntok=4) == _lib.WKV_ERR_INVALID
    # nothing to attend: a no-op success
    assert call(batch=0) == _lib.WKV_OK
    assert call(mq=0) == _lib.WKV_OK


@host_only
def test_grouped_decode_rejects_bad_arguments_before_launch():
    lib = _lib.load()
    d = _desc()
    base = dict(q=16, qsb=1024, qsh=128, out=16, hq=8, bt=16, bts=4, mb=4, sl=16, batch=8, ms=64, pre=16, gs=4,
                mpl=32, scale=0.1, part=0)

    def call(**kw):
        a = dict(base, **kw)
        return lib.wkv_paged_decode_gqa_grouped(ctypes.byref(d), None, 0, 0, None, 0, 0, None, a["q"], a["qsb"],
                                                a["qsh"], a["out"], a["hq"], a["bt"], a["bts"], a["mb"], a["sl"],
                                                a["batch"], a["ms"], a["pre"], a["gs"], a["mpl"], a["scale"],
                                                a["part"], None, 0, None, None)

    assert call(hq=3) == _lib.WKV_ERR_INVALID
    assert call(hq=64) == _lib.WKV_ERR_UNSUPPORTED  # 32 query heads per KV head
    assert call(pre=None) == _lib.WKV_ERR_INVALID
    assert "prefix_lens" in _lib.last_error()
    assert call(gs=0) == _lib.WKV_ERR_INVALID
    assert call(gs=9) == _lib.WKV_ERR_INVALID  # group larger than the batch
    assert call(mpl=-1) == _lib.WKV_ERR_INVALID
    assert call(part=24) == _lib.WKV_ERR_INVALID  # not a multiple of the block size
    assert call(scale=float("nan")) == _lib.WKV_ERR_INVALID
    assert call(bt=None) == _lib.WKV_ERR_INVALID


@host_only
def test_sample_gather_copy_reject_bad_arguments_before_launch():
    lib = _lib.load()
    s = lib.wkv_sample

    def sample(logits=16, dtype=1, stride=1024, batch=2, vocab=1024, out=16):
        return s(logits, dtype, stride, batch, vocab, None, None, None, None, None, None, None, 0, out, None, None,
                 None, None)

    assert sample(vocab=0) == _lib.WKV_ERR_INVALID
    assert sample(logits=None) == _lib.WKV_ERR_INVALID
    assert sample(out=None) == _lib.WKV_ERR_INVALID
    assert sample(dtype=2) == _lib.WKV_ERR_INVALID
    assert sample(stride=1000) == _lib.WKV_ERR_INVALID  # rows shorter than the vocabulary
    assert sample(batch=0) == _lib.WKV_OK
    d = _desc()
    g = lib.wkv_gather

    def gather(bt=16, bts=4, mb=4, sl=16, cu=16, batch=2, ok=16, ov=16, dq=0):
        return g(ctypes.byref(d), bt, bts, mb, sl, cu, batch, ok, ov, dq, None)

    assert gather(batch=-1) == _lib.WKV_ERR_INVALID
    assert gather(bts=2) == _lib.WKV_ERR_INVALID
    assert gather(bt=None) == _lib.WKV_ERR_INVALID
    assert gather(ok=17) == _lib.WKV_ERR_INVALID
    assert gather(dq=2) == _lib.WKV_ERR_INVALID
    assert gather(dq=1) == _lib.WKV_ERR_INVALID  # dequantizing applies to fp8 caches only
    assert gather(batch=0) == _lib.WKV_OK
    assert lib.wkv_copy_blocks(ctypes.byref(d), None, -1, None) == _lib.WKV_ERR_INVALID
    assert lib.wkv_copy_blocks(ctypes.byref(d), None, 1, None) == _lib.WKV_ERR_INVALID
    assert lib.wkv_copy_blocks(ctypes.byref(d), None, 0, None) == _lib.WKV_OK


@host_only
def test_cache_descriptor_flags_and_reserved_are_checked():
    """Unknown flag bits and a non-zero `reserved` are refused (wkv.h documents both),
    so a caller built against an older or newer descriptor cannot pass garbage."""
    lib = _lib.load()
    for kw in (dict(flags=2), dict(flags=-1), dict(reserved=1)):
        d = _desc(**kw)
        assert lib.wkv_copy_blocks(ctypes.byref(d), 16, 1, None) == _lib.WKV_ERR_INVALID
        assert "flags" in _lib.last_error() or "reserved" in _lib.last_error()
    d = _desc(flags=_lib.CACHE_SHARED_BLOCKS)
    assert lib.wkv_copy_blocks(ctypes.byref(d), 16, 0, None) == _lib.WKV_OK


@host_only
def test_mla_gather_copy_and_sinks_reject_bad_arguments_before_launch():
    lib = _lib.load()
    m = _lib.WkvMlaCache(latent=16, num_blocks=4, block_size=64, kv_lora_rank=512, rope_dim=64)
    g = lib.wkv_mla_gather

    def gather(bt=16, bts=4, mb=4, sl=16, cu=16, batch=2, out=16, cache=m):
        return g(ctypes.byref(cache), bt, bts, mb, sl, cu, batch, out, None)

    assert gather(batch=-1) == _lib.WKV_ERR_INVALID
    assert gather(bts=2) == _lib.WKV_ERR_INVALID
    assert gather(bt=None) == _lib.WKV_ERR_INVALID
    assert gather(cu=None) == _lib.WKV_ERR_INVALID
    assert gather(out=None) == _lib.WKV_ERR_INVALID
    assert gather(out=24) == _lib.WKV_ERR_INVALID  # not 16-byte aligned
    assert gather(batch=0) == _lib.WKV_OK
    bad = _lib.WkvMlaCache(latent=16, num_blocks=4, block_size=40, kv_lora_rank=512, rope_dim=64)
    assert gather(cache=bad) == _lib.WKV_ERR_INVALID
    assert lib.wkv_mla_gather(None, 16, 4, 4, 16, 16, 2, 16, None) == _lib.WKV_ERR_INVALID
    c = lib.wkv_mla_copy_blocks
    assert c(ctypes.byref(m), None, -1, None) == _lib.WKV_ERR_INVALID
    assert c(ctypes.byref(m), None, 1, None) == _lib.WKV_ERR_INVALID
    assert c(ctypes.byref(m), None, 0, None) == _lib.WKV_OK
    assert c(ctypes.byref(bad), 16, 1, None) == _lib.WKV_ERR_INVALID
    # sinks: NULL or misaligned sinks refused; otherwise the plain call's checks
    d = lib.wkv_paged_decode_mla_sinks
    args = (16, 0, 0, 16, 0, 0, 16, 128, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0)
    assert d(ctypes.byref(m), *args, None, None) == _lib.WKV_ERR_INVALID
    assert d(ctypes.byref(m), *args, 18, None) == _lib.WKV_ERR_INVALID
    m256 = _lib.WkvMlaCache(latent=16, num_blocks=4, block_size=64, kv_lora_rank=256, rope_dim=64)
    assert d(ctypes.byref(m256), *args, 16, None) == _lib.WKV_ERR_UNSUPPORTED
    f = lib.wkv_append_paged_decode_mla_sinks
    fargs = (16, 512, 16, 64, 16, 16, 0, 0, 16, 0, 0, 16, 128, 16, 1, 1, 16, 1, 64, 0.1, 0, None, 0)
    assert f(ctypes.byref(m), *fargs, None, None) == _lib.WKV_ERR_INVALID
    assert f(ctypes.byref(m), None, *fargs[1:], 16, None) == _lib.WKV_ERR_INVALID
    assert f(ctypes.byref(m), 16, 512, 16, 64, None, *fargs[5:], 16, None) == _lib.WKV_ERR_INVALID
