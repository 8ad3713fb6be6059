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
    assert lib.wkv_mla_workspace_size(32, 128, 512, 4096, 512) == 32 * 128 * 8 * 514 * 4


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
