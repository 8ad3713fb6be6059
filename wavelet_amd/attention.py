"""Paged decode attention over ``PagedKVCache`` / ``MLALatentCache``.

The attention half of the engine's KV surface: for each decode step the
reference's engine runs, per layer, ``softmax(q . K^T * scale) . V`` over each
sequence's context read through its block table (inside ``llm.generate``,
wavelet/inference/engine.py:887; semantics of ``_eager_sparse_attention``,
wavelet/trainer/models/deepseek_v4/attention.py:81-96, and of the
``attention_interface(..., scaling=self.scaling)`` call at
wavelet/kernels/patch.py:182-196).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .cache import MLALatentCache, PagedKVCache, _require_cuda, _slots, _stream, _token_rows, check_tables

_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def _key(device: torch.device) -> tuple[int, int]:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return idx, torch.cuda.current_stream(device).cuda_stream


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-(device, stream) scratch for split-K partials, grown on demand and reused."""
    key = _key(device)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _query(q: torch.Tensor, name: str, shape: tuple[int, ...], device: torch.device) -> torch.Tensor:
    _require_cuda(q, name, device)
    if q.dtype != torch.bfloat16 or q.dim() != 3 or tuple(q.shape[1:]) != shape:
        raise ValueError(f"{name} must be bfloat16 [B, {', '.join(map(str, shape))}] (got {q.dtype} {tuple(q.shape)})")
    if q.stride(2) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    return q


def _order(seq_order: torch.Tensor | None, batch: int, dev: torch.device) -> int | None:
    """The device pointer of a dispatch order (None = batch order), checked."""
    if seq_order is None:
        return None
    if (seq_order.dtype != torch.int32 or tuple(seq_order.shape) != (batch,) or not seq_order.is_contiguous()
            or seq_order.device != dev):
        raise ValueError(f"seq_order must be a contiguous int32 [{batch}] tensor on {dev}")
    return seq_order.data_ptr()


def _max_len(seq_lens: torch.Tensor, max_seq_len: int | None) -> int:
    if max_seq_len is not None:
        return int(max_seq_len)
    return int(seq_lens.max().item()) if seq_lens.numel() else 0


def decode_plan(batch: int, num_kv_heads: int, max_seq_len: int, block_size: int,
                partition_size: int = 0) -> tuple[int, int, int]:
    """(partition size, waves per workgroup, workgroups per sequence and KV head)
    that ``paged_decode_gqa`` launches for this geometry (host-side, no GPU)."""
    p, w, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    _lib.check(_lib.load().wkv_decode_plan(int(batch), int(num_kv_heads), int(max_seq_len), int(block_size),
                                           int(partition_size), ctypes.byref(p), ctypes.byref(w), ctypes.byref(c)),
               "decode_plan")
    return p.value, w.value, c.value


def decode_order(seq_lens: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Dispatch order for ``paged_decode_gqa``: int32 ``[B]`` sequence indices by
    ``seq_lens``, longest first, ties by index (computed on the device).

    A decode launch lasts as long as its last workgroups; dispatching the long
    contexts first lets the short ones fill in behind them. The order depends
    only on the lengths, so one call per step serves every layer.
    """
    if seq_lens.dtype != torch.int32 or seq_lens.dim() != 1 or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 vector")
    batch = seq_lens.shape[0]
    if out is None:
        out = torch.empty(batch, dtype=torch.int32, device=seq_lens.device)
    elif (out.dtype != torch.int32 or tuple(out.shape) != (batch,) or not out.is_contiguous()
          or out.device != seq_lens.device):
        raise ValueError(f"out must be a contiguous int32 [{batch}] tensor on {seq_lens.device}")
    _lib.check(_lib.load().wkv_decode_order(seq_lens.data_ptr(), batch, out.data_ptr(), _stream(seq_lens.device)),
               "decode_order")
    return out


def grouped_decode_order(seq_lens: torch.Tensor, group_size: int, num_kv_heads: int, max_seq_len: int,
                         block_size: int, partition_size: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Dispatch order for ``paged_decode_gqa_grouped`` (GRPO groups of ``group_size``
    consecutive sequences): longest first within classes of whole groups that the
    decode launch maps to the same XCDs, the classes interleaved, so that a group's
    members read its prompt through one L2 (``decode_order`` when the classes cannot
    be of equal size). The geometry is the one the grouped decode calls will get."""
    if seq_lens.dtype != torch.int32 or seq_lens.dim() != 1 or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 vector")
    batch = seq_lens.shape[0]
    if out is None:
        out = torch.empty(batch, dtype=torch.int32, device=seq_lens.device)
    elif (out.dtype != torch.int32 or tuple(out.shape) != (batch,) or not out.is_contiguous()
          or out.device != seq_lens.device):
        raise ValueError(f"out must be a contiguous int32 [{batch}] tensor on {seq_lens.device}")
    _lib.check(_lib.load().wkv_grouped_decode_order(seq_lens.data_ptr(), batch, int(group_size), int(num_kv_heads),
                                                     int(max_seq_len), int(block_size), int(partition_size),
                                                     out.data_ptr(), _stream(seq_lens.device)),
               "grouped_decode_order")
    return out


def paged_decode_gqa(
    q: torch.Tensor,
    cache: PagedKVCache,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float,
    *,
    max_seq_len: int | None = None,
    out: torch.Tensor | None = None,
    partition_size: int = 0,
    new_key: torch.Tensor | None = None,
    new_value: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
    seq_order: torch.Tensor | None = None,
    sinks: torch.Tensor | None = None,
    shared_blocks: bool | None = None,
) -> torch.Tensor:
    """One decode step of GQA attention: ``q [B, Hq, D]`` bf16 -> ``[B, Hq, D]`` bf16.

    Query head ``h`` reads KV head ``h // (Hq // Hkv)``. ``max_seq_len`` (a host
    int, >= every ``seq_lens``) avoids a device sync when given. With
    ``new_key``/``new_value`` ``[B, Hkv, D]`` and ``slot_mapping [B]`` the step's
    append is fused into the same launch: token ``b`` is written at
    ``slot_mapping[b]`` (position ``seq_lens[b] - 1`` of sequence ``b``) before
    attention reads it -- the same result as ``cache.append`` then this call.
    ``seq_order`` (int32 ``[B]``, a permutation of ``0..B-1``, e.g. from
    ``decode_order``) sets the order in which sequences are dispatched; the
    result is the same, bit for bit, in any order. ``sinks`` (fp32 ``[Hq]``,
    natural-log logits, ``-inf`` = none) adds one zero-value logit per query
    head to its softmax: the learned sink of the reference's sparse attention
    (wavelet/trainer/models/deepseek_v4/attention.py:89-95). ``shared_blocks``
    is this step's read policy (None = the cache's default): True when some
    block is read by more than one sequence of the step (K/V reads then keep
    it cached for the next reader), False to stream every block past the
    caches (``KVPool.decode_shares_blocks`` decides it from the step's tables).
    """
    if not isinstance(cache, PagedKVCache):
        raise ValueError("cache must be a PagedKVCache")
    dev = cache.device
    block_table, seq_lens = check_tables(block_table, seq_lens, dev, cache.block_size)
    batch = seq_lens.shape[0]
    if q.dim() != 3 or q.shape[0] != batch:
        raise ValueError(f"q must be [B={batch}, Hq, D]")
    hq = q.shape[1]
    q = _query(q, "q", (hq, cache.head_dim), dev)
    fused = new_key is not None or new_value is not None or slot_mapping is not None
    if fused:
        if new_key is None or new_value is None or slot_mapping is None:
            raise ValueError("a fused append needs new_key, new_value and slot_mapping together")
        shape = (cache.num_kv_heads, cache.head_dim)
        new_key = _token_rows(new_key, "new_key", shape, dev)
        new_value = _token_rows(new_value, "new_value", shape, dev)
        if new_key.shape[0] != batch or new_value.shape[0] != batch:
            raise ValueError(f"new_key/new_value must hold one token per sequence ({batch})")
        slot_mapping = _slots(slot_mapping, batch, dev)
    sinks = _sinks(sinks, hq, dev)
    if out is None:
        out = torch.empty((batch, hq, cache.head_dim), dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (batch, hq, cache.head_dim) or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 [B, Hq, D] tensor")
    if batch == 0:
        return out
    lib = _lib.load()
    msl = _max_len(seq_lens, max_seq_len)
    need = lib.wkv_decode_workspace_size(batch, hq, cache.head_dim, max(msl, 1), int(partition_size))
    if need < 0:
        raise ValueError("invalid decode geometry")
    ws = _workspace(dev, need)
    tail = (q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), hq, block_table.data_ptr(),
            block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(), batch, msl, float(scale),
            int(partition_size), ws.data_ptr(), ws.numel(), _order(seq_order, batch, dev))
    tail = tail + ((sinks.data_ptr(),) if sinks is not None else ()) + (_stream(dev),)
    desc = ctypes.byref(cache.descriptor(shared_blocks))
    if fused:
        fn = lib.wkv_append_paged_decode_gqa_sinks if sinks is not None else lib.wkv_append_paged_decode_gqa
        rc = fn(desc, new_key.data_ptr(), new_key.stride(0), new_key.stride(1), new_value.data_ptr(),
                new_value.stride(0), new_value.stride(1), slot_mapping.data_ptr(), *tail)
    else:
        fn = lib.wkv_paged_decode_gqa_sinks if sinks is not None else lib.wkv_paged_decode_gqa
        rc = fn(desc, *tail)
    _lib.check(rc, "paged_decode_gqa")
    return out


def paged_decode_gqa_grouped(
    q: torch.Tensor,
    cache: PagedKVCache,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    prefix_lens: torch.Tensor,
    group_size: int,
    scale: float,
    *,
    max_seq_len: int | None = None,
    max_prefix_len: int | None = None,
    out: torch.Tensor | None = None,
    partition_size: int = 0,
    new_key: torch.Tensor | None = None,
    new_value: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
    seq_order: torch.Tensor | None = None,
) -> torch.Tensor:
    """``paged_decode_gqa`` for GRPO groups, reading their shared prompt through the caches.

    Sequences ``g*group_size .. g*group_size+group_size-1`` form group ``g``;
    ``prefix_lens [n_groups]`` int32 gives the leading tokens whose physical
    blocks every member's table shares (``BlockManager.shared_prefix_tokens``).
    The result is ``paged_decode_gqa``'s on the same inputs, bit for bit (with
    the fused append: ``paged_decode_gqa`` after ``append``); the groups steer
    how the cache is read: the prompt blocks keep the default cache policy, so
    the members' reads of one block meet in the L2 and the last-level cache,
    and each member's own tokens are streamed past them. ``seq_order`` from
    ``grouped_decode_order`` also runs a group's members on one XCD. Optional
    fused append as in ``paged_decode_gqa`` (the group semantics follow
    ``SamplingParams(n=...)``, wavelet/inference/engine.py:69-90).
    """
    if not isinstance(cache, PagedKVCache):
        raise ValueError("cache must be a PagedKVCache")
    dev = cache.device
    block_table, seq_lens = check_tables(block_table, seq_lens, dev, cache.block_size)
    batch = seq_lens.shape[0]
    group_size = int(group_size)
    if group_size < 1 or (batch and group_size > batch):
        raise ValueError(f"group_size must be in [1, batch={batch}] (got {group_size})")
    n_groups = -(-batch // group_size) if batch else 0
    _require_cuda(prefix_lens, "prefix_lens", dev)
    if prefix_lens.dtype != torch.int32 or prefix_lens.dim() != 1 or prefix_lens.shape[0] != n_groups:
        raise ValueError(f"prefix_lens must be int32 [{n_groups}] (got {prefix_lens.dtype} {tuple(prefix_lens.shape)})")
    prefix_lens = prefix_lens.contiguous()
    if q.dim() != 3 or q.shape[0] != batch:
        raise ValueError(f"q must be [B={batch}, Hq, D]")
    hq = q.shape[1]
    q = _query(q, "q", (hq, cache.head_dim), dev)
    fused = new_key is not None or new_value is not None or slot_mapping is not None
    if fused:
        if new_key is None or new_value is None or slot_mapping is None:
            raise ValueError("a fused append needs new_key, new_value and slot_mapping together")
        shape = (cache.num_kv_heads, cache.head_dim)
        new_key = _token_rows(new_key, "new_key", shape, dev)
        new_value = _token_rows(new_value, "new_value", shape, dev)
        if new_key.shape[0] != batch or new_value.shape[0] != batch:
            raise ValueError(f"new_key/new_value must hold one token per sequence ({batch})")
        slot_mapping = _slots(slot_mapping, batch, dev)
    if out is None:
        out = torch.empty((batch, hq, cache.head_dim), dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (batch, hq, cache.head_dim) or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 [B, Hq, D] tensor")
    if batch == 0:
        return out
    lib = _lib.load()
    msl = _max_len(seq_lens, max_seq_len)
    mpl = int(max_prefix_len) if max_prefix_len is not None else (
        int(prefix_lens.max().item()) if prefix_lens.numel() else 0)
    need = lib.wkv_grouped_decode_workspace_size(batch, hq, cache.head_dim, max(msl, 1), max(mpl, 0),
                                                 int(partition_size))
    if need < 0:
        raise ValueError("invalid grouped decode geometry")
    ws = _workspace(dev, need)
    if fused:
        head = (new_key.data_ptr(), new_key.stride(0), new_key.stride(1), new_value.data_ptr(), new_value.stride(0),
                new_value.stride(1), slot_mapping.data_ptr())
    else:
        head = (None, 0, 0, None, 0, 0, None)
    rc = lib.wkv_paged_decode_gqa_grouped(
        ctypes.byref(cache.descriptor()), *head, q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), hq,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(), batch, msl,
        prefix_lens.data_ptr(), group_size, mpl, float(scale), int(partition_size), ws.data_ptr(), ws.numel(),
        _order(seq_order, batch, dev), _stream(dev))
    _lib.check(rc, "paged_decode_gqa_grouped")
    return out


def _sinks(sinks: torch.Tensor | None, hq: int, dev: torch.device) -> torch.Tensor | None:
    """Per-query-head attention sinks: None, or a contiguous float32 [Hq] device tensor."""
    if sinks is None:
        return None
    if not isinstance(sinks, torch.Tensor) or sinks.dtype != torch.float32 or tuple(sinks.shape) != (hq,) \
            or sinks.device != dev:
        raise ValueError(f"sinks must be a float32 [{hq}] tensor on {dev}")
    return sinks.contiguous()


def prefill_gqa(
    q: torch.Tensor,
    cache: PagedKVCache,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    scale: float,
    *,
    key: torch.Tensor | None = None,
    value: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
    max_query_len: int | None = None,
    max_seq_len: int | None = None,
    out: torch.Tensor | None = None,
    sinks: torch.Tensor | None = None,
) -> torch.Tensor:
    """Varlen (chunked) prefill: ``q [T, Hq, D]`` bf16 -> ``[T, Hq, D]`` bf16.

    Sequence ``b`` owns rows ``cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1`` (int32
    ``[B+1]``), new tokens at positions ``seq_lens[b] - n_b ..`` of a context
    of ``seq_lens[b]`` tokens (earlier chunks / prefix-cache hits are cached
    context); token ``j`` attends causally to positions ``0 .. seq_lens[b] -
    n_b + j``. With ``key``/``value`` ``[T, Hkv, D]`` and ``slot_mapping [T]``
    the new tokens are appended first (``cache.append``) and attended from the
    cache -- the prompt step of ``llm.generate`` (wavelet/inference/
    engine.py:887). ``max_query_len`` / ``max_seq_len`` (host ints) avoid
    device syncs when given. ``sinks`` as for ``paged_decode_gqa``.
    """
    if not isinstance(cache, PagedKVCache):
        raise ValueError("cache must be a PagedKVCache")
    dev = cache.device
    block_table, seq_lens = check_tables(block_table, seq_lens, dev, cache.block_size)
    batch = seq_lens.shape[0]
    _require_cuda(cu_seqlens_q, "cu_seqlens_q", dev)
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_q.dim() != 1 or cu_seqlens_q.shape[0] != batch + 1:
        raise ValueError(f"cu_seqlens_q must be int32 [{batch + 1}]")
    cu_seqlens_q = cu_seqlens_q.contiguous()
    if q.dim() != 3:
        raise ValueError("q must be [T, Hq, D]")
    tokens, hq = q.shape[0], q.shape[1]
    q = _query(q, "q", (hq, cache.head_dim), dev)
    append = key is not None or value is not None or slot_mapping is not None
    if append:
        if key is None or value is None or slot_mapping is None:
            raise ValueError("appending needs key, value and slot_mapping together")
        shape = (cache.num_kv_heads, cache.head_dim)
        key = _token_rows(key, "key", shape, dev)
        value = _token_rows(value, "value", shape, dev)
        if key.shape[0] != tokens or value.shape[0] != tokens:
            raise ValueError(f"key/value must hold the {tokens} new tokens")
        slot_mapping = _slots(slot_mapping, tokens, dev)
    if out is None:
        out = torch.empty((tokens, hq, cache.head_dim), dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (tokens, hq, cache.head_dim) or out.stride(2) != 1:
        raise ValueError("out must be a bfloat16 [T, Hq, D] tensor with a contiguous last dim")
    sinks = _sinks(sinks, hq, dev)
    if max_query_len is None:
        max_query_len = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item()) if batch else 0
    msl = _max_len(seq_lens, max_seq_len)
    lib = _lib.load()
    if append:
        head = (key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0), value.stride(1),
                slot_mapping.data_ptr(), tokens)
    else:
        head = (None, 0, 0, None, 0, 0, None, 0)
    args = (ctypes.byref(cache.descriptor()), *head, q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(),
            out.stride(0), out.stride(1), hq, cu_seqlens_q.data_ptr(), seq_lens.data_ptr(), block_table.data_ptr(),
            block_table.stride(0), block_table.shape[1], batch, int(max_query_len), msl, float(scale))
    if sinks is not None:
        rc = lib.wkv_prefill_gqa_sinks(*args, sinks.data_ptr(), _stream(dev))
    else:
        rc = lib.wkv_prefill_gqa(*args, _stream(dev))
    _lib.check(rc, "prefill_gqa")
    return out


def paged_decode_mla(
    q_nope: torch.Tensor,
    q_pe: torch.Tensor,
    cache: MLALatentCache,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float,
    *,
    max_seq_len: int | None = None,
    out: torch.Tensor | None = None,
    partition_size: int = 0,
    new_kv_c: torch.Tensor | None = None,
    new_k_pe: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
    sinks: torch.Tensor | None = None,
) -> torch.Tensor:
    """Weight-absorbed MLA decode: ``q_nope [B, H, R]``, ``q_pe [B, H, P]`` -> ``[B, H, R]`` bf16.

    With ``new_kv_c [B, R]``, ``new_k_pe [B, P]`` and ``slot_mapping [B]`` the
    step's latent append is fused into the same launch: token ``b`` is written
    at ``slot_mapping[b]`` (position ``seq_lens[b] - 1`` of sequence ``b``) and
    attended -- the same result as ``cache.append`` then this call. ``sinks``
    (fp32 ``[H]``, natural-log logits, ``-inf`` = none) adds one zero-value
    logit per head to its softmax: the learned per-head sink of the
    reference's shared-KV attention (wavelet/trainer/models/deepseek_v4/
    attention.py:703, consumed at :89-95 and :763).
    """
    if not isinstance(cache, MLALatentCache):
        raise ValueError("cache must be an MLALatentCache")
    dev = cache.device
    block_table, seq_lens = check_tables(block_table, seq_lens, dev, cache.block_size)
    batch = seq_lens.shape[0]
    if q_nope.dim() != 3 or q_nope.shape[0] != batch:
        raise ValueError(f"q_nope must be [B={batch}, H, {cache.kv_lora_rank}]")
    heads = q_nope.shape[1]
    q_nope = _query(q_nope, "q_nope", (heads, cache.kv_lora_rank), dev)
    q_pe = _query(q_pe, "q_pe", (heads, cache.rope_dim), dev)
    if q_pe.shape[0] != batch:
        raise ValueError("q_pe batch differs from q_nope")
    fused = new_kv_c is not None or new_k_pe is not None or slot_mapping is not None
    if fused:
        if new_kv_c is None or new_k_pe is None or slot_mapping is None:
            raise ValueError("a fused append needs new_kv_c, new_k_pe and slot_mapping together")
        rows = []
        for name, x, w in (("new_kv_c", new_kv_c, cache.kv_lora_rank), ("new_k_pe", new_k_pe, cache.rope_dim)):
            _require_cuda(x, name, dev)
            if x.dtype != torch.bfloat16 or x.dim() != 2 or tuple(x.shape) != (batch, w):
                raise ValueError(f"{name} must be bfloat16 [{batch}, {w}]")
            if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
                x = x.contiguous()
            rows.append(x)
        new_kv_c, new_k_pe = rows
        slot_mapping = _slots(slot_mapping, batch, dev)
    sinks = _sinks(sinks, heads, dev)
    if out is None:
        out = torch.empty((batch, heads, cache.kv_lora_rank), dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (batch, heads, cache.kv_lora_rank) or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 [B, H, R] tensor")
    if batch == 0:
        return out
    lib = _lib.load()
    msl = _max_len(seq_lens, max_seq_len)
    need = lib.wkv_mla_workspace_size(batch, heads, cache.kv_lora_rank, max(msl, 1), int(partition_size))
    if need < 0:
        raise ValueError("invalid MLA decode geometry")
    ws = _workspace(dev, need)
    tail = (q_nope.data_ptr(), q_nope.stride(0), q_nope.stride(1), q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1),
            out.data_ptr(), heads, block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            seq_lens.data_ptr(), batch, msl, float(scale), int(partition_size), ws.data_ptr(), ws.numel())
    tail = tail + ((sinks.data_ptr(),) if sinks is not None else ()) + (_stream(dev),)
    if fused:
        fn = lib.wkv_append_paged_decode_mla_sinks if sinks is not None else lib.wkv_append_paged_decode_mla
        rc = fn(ctypes.byref(cache.descriptor()), new_kv_c.data_ptr(), new_kv_c.stride(0), new_k_pe.data_ptr(),
                new_k_pe.stride(0), slot_mapping.data_ptr(), *tail)
    else:
        fn = lib.wkv_paged_decode_mla_sinks if sinks is not None else lib.wkv_paged_decode_mla
        rc = fn(ctypes.byref(cache.descriptor()), *tail)
    _lib.check(rc, "paged_decode_mla")
    return out
