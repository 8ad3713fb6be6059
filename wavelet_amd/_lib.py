"""ctypes binding of libwkv.so (declarations in include/wkv.h).

The product path has no fallback: if the library is missing or fails to load,
every entry point raises. Status codes map to the reference's error idiom
(wavelet/inference/engine.py:191-233, :772-774): argument errors raise
ValueError, unsupported shapes NotImplementedError, launch failures
RuntimeError, each carrying the library's thread-local message.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwkv.so"

WKV_OK, WKV_ERR_INVALID, WKV_ERR_UNSUPPORTED, WKV_ERR_LAUNCH = 0, 1, 2, 3
WKV_KV_BF16, WKV_KV_FP8_E4M3 = 0, 1
WKV_NOALLOC_SCRATCH_BYTES = 32 << 20  # include/wkv.h


# wkv_cache_t.flags: several sequences read the same blocks (prefix caching)
CACHE_SHARED_BLOCKS = 1


class WkvCache(ctypes.Structure):
    _fields_ = [
        ("k", c_void_p),
        ("v", c_void_p),
        ("k_scale", c_void_p),
        ("v_scale", c_void_p),
        ("num_blocks", c_int64),
        ("block_size", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("kv_dtype", c_int32),
        ("flags", c_int32),
        ("reserved", c_int32),
    ]


class WkvMlaCache(ctypes.Structure):
    _fields_ = [
        ("latent", c_void_p),
        ("num_blocks", c_int64),
        ("block_size", c_int32),
        ("kv_lora_rank", c_int32),
        ("rope_dim", c_int32),
    ]


_I64P = POINTER(c_int64)
_SIGNATURES = {
    "wkv_append": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "wkv_append_fp8": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "wkv_mla_append": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "wkv_gather": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_void_p]),
    "wkv_copy_blocks": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_void_p]),
    "wkv_mla_gather": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p]),
    "wkv_mla_copy_blocks": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_void_p]),
    "wkv_decode_workspace_size": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "wkv_decode_order": (c_int, [c_void_p, c_int32, c_void_p, c_void_p]),
    "wkv_grouped_decode_order": (c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p,
                                         c_void_p]),
    "wkv_decode_plan": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, POINTER(c_int32), POINTER(c_int32), POINTER(c_int32)]),
    "wkv_paged_decode_gqa": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p]),
    "wkv_append_paged_decode_gqa": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p]),
    "wkv_paged_decode_gqa_sinks": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "wkv_append_paged_decode_gqa_sinks": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "wkv_append_paged_decode_gqa_noalloc": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_void_p]),
    "wkv_grouped_decode_workspace_size": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "wkv_paged_decode_gqa_grouped": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p]),
    "wkv_prefill_gqa": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_float, c_void_p]),
    "wkv_prefill_gqa_sinks": (c_int, [POINTER(WkvCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_float, c_void_p, c_void_p]),
    "wkv_sample": (c_int, [c_void_p, c_int32, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "wkv_mla_workspace_size": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "wkv_paged_decode_mla": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p]),
    "wkv_append_paged_decode_mla": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p]),
    "wkv_paged_decode_mla_sinks": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p]),
    "wkv_append_paged_decode_mla_sinks": (c_int, [POINTER(WkvMlaCache), c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32, c_float, c_int32, c_void_p, c_int64, c_void_p, c_void_p]),
    "wkv_hbm_read_probe": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p]),
    "wkv_last_error": (c_char_p, []),
    "wkv_version": (c_int, []),
}

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libwkv.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library with `python -m wavelet_amd.build` "
                "(there is no CPU fallback for the KV path)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().wkv_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc == WKV_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == WKV_ERR_INVALID:
        raise ValueError(msg)
    if rc == WKV_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
