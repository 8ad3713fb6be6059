"""MI355X-native paged KV-cache decode path (gfx950 HIP kernels behind a C ABI).

Public surface (a drop-in for the KV path of the reference's inference engine):

* ``PagedKVCache`` / ``MLALatentCache`` -- per-layer caches with ``append``,
  ``gather`` and ``copy_blocks``;
* ``paged_decode_gqa`` / ``paged_decode_mla`` -- one decode step of attention;
  ``decode_order`` -- a step's longest-first dispatch order for the former,
  ``decode_plan`` -- its launch shape;
* ``paged_decode_gqa_grouped`` -- the same for GRPO groups, reading each
  group's shared prompt blocks through the caches and the members' own tokens
  streamed; ``grouped_decode_order`` -- its dispatch order;
* ``prefill_gqa`` -- varlen (chunked) prefill that appends the prompt's K/V
  and attends causally over the paged context;
* ``BlockManager`` -- host-side block allocation with ref-counted prefix
  sharing for GRPO groups;
* ``KVPool`` -- all layers' caches plus the block manager, with the engine's
  sleep / wake_up lifecycle and KV metrics;
* ``sample`` -- the token sampler after decode (temperature, min_p, top_k,
  top_p, repetition penalty; processed logprobs and the sampling mask).

Also, by module: ``wavelet_amd.plan`` -- a whole decode or prompt step over
every layer, built once and launched per step (``DecodeStep``,
``MLADecodeStep``, ``PrefillStep``), and ``GraphDecodeStep``, the decode step
captured in one HIP graph; ``wavelet_amd.hf`` -- a transformers ``Cache`` over
a ``KVPool`` and the ``"wavelet_paged"`` attention implementation.
"""

from .attention import (decode_order, decode_plan, grouped_decode_order, paged_decode_gqa, paged_decode_gqa_grouped,
                        paged_decode_mla, prefill_gqa)
from .blocks import BlockManager
from .cache import MLALatentCache, PagedKVCache, validate_group_prefix, validate_tables
from .pool import KVPool
from .sampler import sample

__all__ = [
    "BlockManager",
    "KVPool",
    "MLALatentCache",
    "PagedKVCache",
    "decode_order",
    "grouped_decode_order",
    "decode_plan",
    "paged_decode_gqa",
    "paged_decode_gqa_grouped",
    "paged_decode_mla",
    "prefill_gqa",
    "sample",
    "validate_group_prefix",
    "validate_tables",
]
