"""Pre-validated decode-step launch plans.

A serving loop calls append + attention once per layer per decode step with
buffers whose shapes never change between steps. ``DecodeStep`` validates
those buffers once, resolves every pointer, stride and workspace, and then
replays the C-ABI calls directly -- two ctypes calls per layer and no tensor
inspection -- so host overhead stays far below the GPU time of a step.
The tensors handed to it must stay alive (and keep their storage) for the
plan's lifetime; refill them in place between steps.

A plan holds the raw pointers of its caches. ``KVPool.sleep`` /
``PagedKVCache.sleep`` free that memory and ``wake_up`` allocates new memory,
so a plan built before a sleep refuses to launch afterwards (RuntimeError):
build a new plan after ``wake_up``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .attention import _workspace, decode_plan
from .cache import PagedKVCache, _require_cuda, check_tables


# Smallest B * Hkv * max_seq_len (token-heads) for which DecodeStep orders
# its dispatch by default.
ORDER_MIN_WORK = 1 << 20


def _plan_slots(slot_mapping: torch.Tensor, device: torch.device, n: int | None) -> torch.Tensor:
    """A plan's slot mapping: contiguous int64 on the caches' device, ``n`` entries when given."""
    _require_cuda(slot_mapping, "slot_mapping", device)
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be a contiguous int64 vector")
    if n is not None and slot_mapping.numel() != n:
        raise ValueError(f"slot_mapping must hold one slot per sequence ({n}), got {slot_mapping.numel()}")
    return slot_mapping


class _Live:
    """The cache descriptors a plan was built on; launching is refused once any
    cache has been released or re-allocated (sleep / wake_up)."""

    def __init__(self, caches) -> None:
        self._pairs = [(c, c.descriptor()) for c in caches]

    def check(self, layer: int) -> None:
        cache, desc = self._pairs[layer]
        if cache._desc is not desc:
            state = "asleep" if cache._desc is None else "re-allocated by wake_up"
            raise RuntimeError(f"layer {layer}: the KV cache this plan was built on is {state}; build a new plan")

    def check_all(self) -> None:
        for layer in range(len(self._pairs)):
            self.check(layer)


@dataclass
class _LayerCall:
    append_fn: object
    append_args: tuple
    decode_args: dict  # read policy (shared_blocks) -> the attention call's arguments
    fused_args: dict   # read policy -> the fused append + attention call's arguments
    shared_default: bool


class DecodeStep:
    """Append one token per sequence, then GQA decode attention, for every layer.

    ``caches[l]`` is layer ``l``'s cache; ``q[l]`` ``[B, Hq, D]``, ``key[l]`` /
    ``value[l]`` ``[T, Hkv, D]`` and ``out[l]`` ``[B, Hq, D]`` are the per-layer
    step buffers; ``block_table`` / ``seq_lens`` / ``slot_mapping`` are shared by
    all layers (as in a paged engine, one table per sequence). ``slot_mapping[b]``
    is the slot of sequence ``b``'s new token (one token per sequence).

    With ``group_size`` and ``prefix_lens`` (int32 ``[n_groups]`` on the device)
    the attention is the group-aware one (``paged_decode_gqa_grouped``): GRPO
    groups of ``group_size`` consecutive sequences read their shared prompt
    blocks through the caches and their own tokens streamed; ``max_prefix_len``
    bounds ``prefix_lens``.

    With ``order_by_length``, ``run`` first computes the step's dispatch order
    (``decode_order``: longest contexts first; for groups ``grouped_decode_order``,
    which also keeps a group's members on one XCD; one launch shared by every
    layer) and each layer's decode dispatches its sequences in that order; the
    results are the same bit for bit. ``None`` (the default) orders
    when ``B * Hkv * max_seq_len >= 2**20``: below that a launch is short
    enough (~50 us) that the order's dependent read at each workgroup's start
    costs more than mixed lengths lose. Calling ``step_layer`` / ``attend``
    directly uses the order of the last ``prepare`` (the batch order before
    the first).

    ``run``, ``attend`` and ``step_layer`` take the step's read policy
    ``shared_blocks`` (None = each cache's default): True when some block of
    the step is read by more than one sequence (K/V reads keep it cached for
    the next reader), False to stream every block (``KVPool.decode_shares_blocks``
    computes it from the block manager's reference counts once per step). The
    group-aware decode sets its own: each group's prompt cached, the members' own
    tokens streamed.
    """

    def __init__(self, caches: list[PagedKVCache], q: list[torch.Tensor], key: list[torch.Tensor],
                 value: list[torch.Tensor], out: list[torch.Tensor], block_table: torch.Tensor,
                 seq_lens: torch.Tensor, slot_mapping: torch.Tensor, scale: float, max_seq_len: int,
                 partition_size: int = 0, *, group_size: int = 0, prefix_lens: torch.Tensor | None = None,
                 max_prefix_len: int = 0, order_by_length: bool | None = None) -> None:
        if not caches:
            raise ValueError("no layers")
        dev = caches[0].device
        c0 = caches[0]
        self.block_table, self.seq_lens = check_tables(block_table, seq_lens, dev, c0.block_size, strict=True)
        batch = self.seq_lens.shape[0]
        self.slot_mapping = slot_mapping = _plan_slots(slot_mapping, dev, batch)
        if not len(q) == len(key) == len(value) == len(out) == len(caches):
            raise ValueError("q, key, value and out need one tensor per layer")
        self._live = _Live(caches)
        lib = _lib.load()
        hq = q[0].shape[1]
        self.grouped = group_size > 0
        self.group_size = int(group_size)
        if self.grouped:
            n_groups = -(-batch // group_size)
            if (prefix_lens is None or prefix_lens.dtype != torch.int32 or tuple(prefix_lens.shape) != (n_groups,)
                    or not prefix_lens.is_contiguous() or prefix_lens.device != dev):
                raise ValueError(f"prefix_lens must be a contiguous int32 [{n_groups}] tensor on {dev}")
            self.prefix_lens = prefix_lens
            need = lib.wkv_grouped_decode_workspace_size(batch, hq, c0.head_dim, max_seq_len, int(max_prefix_len),
                                                         int(partition_size))
        else:
            need = lib.wkv_decode_workspace_size(batch, hq, c0.head_dim, max_seq_len, int(partition_size))
        if need < 0:
            raise ValueError("invalid decode geometry")
        self.workspace = _workspace(dev, need)
        self.stream = torch.cuda.current_stream(dev).cuda_stream
        self.lib = lib
        if order_by_length is None:
            order_by_length = batch * c0.num_kv_heads * max_seq_len >= ORDER_MIN_WORK
        self.ordered = bool(order_by_length)
        # always a permutation of the batch: the identity until prepare() runs
        self.order = torch.arange(batch, dtype=torch.int32, device=dev)
        order_ptr = self.order.data_ptr() if self.ordered else None
        self.calls: list[_LayerCall] = []
        for layer, cache in enumerate(caches):
            qq, kk, vv, oo = q[layer], key[layer], value[layer], out[layer]
            for name, t, shape in (("q", qq, (batch, hq, cache.head_dim)), ("out", oo, (batch, hq, cache.head_dim)),
                                   ("key", kk, (slot_mapping.numel(), cache.num_kv_heads, cache.head_dim)),
                                   ("value", vv, (slot_mapping.numel(), cache.num_kv_heads, cache.head_dim))):
                if t.dtype != torch.bfloat16 or tuple(t.shape) != shape or not t.is_contiguous() or t.device != dev:
                    raise ValueError(f"layer {layer}: {name} must be a contiguous bfloat16 {shape} tensor on {dev}")
            fn = lib.wkv_append_fp8 if cache.kv_dtype == "fp8_e4m3" else lib.wkv_append
            append_args = (ctypes.byref(cache.descriptor()), kk.data_ptr(), kk.stride(0), kk.stride(1),
                           vv.data_ptr(), vv.stride(0), vv.stride(1), slot_mapping.data_ptr(), slot_mapping.numel(),
                           self.stream)
            tail = (qq.data_ptr(), qq.stride(0), qq.stride(1), oo.data_ptr(), hq,
                    self.block_table.data_ptr(), self.block_table.stride(0), self.block_table.shape[1],
                    self.seq_lens.data_ptr(), batch, int(max_seq_len), ctypes.c_float(scale),
                    int(partition_size), self.workspace.data_ptr(), self.workspace.numel(), self.stream)
            new_kv = (kk.data_ptr(), kk.stride(0), kk.stride(1), vv.data_ptr(), vv.stride(0), vv.stride(1),
                      slot_mapping.data_ptr())
            decode_args, fused_args = {}, {}
            for shared in (False, True):
                desc = ctypes.byref(cache.descriptor(shared))
                if self.grouped:
                    gtail = (*tail[:11], self.prefix_lens.data_ptr(), int(group_size), int(max_prefix_len),
                             *tail[11:-1], order_ptr, tail[-1])
                    decode_args[shared] = (desc, None, 0, 0, None, 0, 0, None, *gtail)
                    fused_args[shared] = (desc, *new_kv, *gtail)
                else:
                    otail = (*tail[:-1], order_ptr, tail[-1])
                    decode_args[shared] = (desc, *otail)
                    fused_args[shared] = (desc, *new_kv, *otail)
            self.calls.append(_LayerCall(fn, append_args, decode_args, fused_args, cache.shared_blocks))
        self._keep = (caches, q, key, value, out)
        self.scale, self.max_seq_len, self.partition_size = float(scale), int(max_seq_len), int(partition_size)

    def prepare(self) -> None:
        """Compute this step's dispatch order from ``seq_lens`` (one launch)."""
        self._live.check_all()
        if self.ordered:
            if self.grouped:
                c0 = self._keep[0][0]
                rc = self.lib.wkv_grouped_decode_order(
                    self.seq_lens.data_ptr(), self.seq_lens.shape[0], self.group_size, c0.num_kv_heads,
                    min(self.max_seq_len, self.block_table.shape[1] * c0.block_size), c0.block_size,
                    self.partition_size, self.order.data_ptr(), self.stream)
            else:
                rc = self.lib.wkv_decode_order(self.seq_lens.data_ptr(), self.seq_lens.shape[0],
                                               self.order.data_ptr(), self.stream)
            if rc:
                _lib.check(rc, "decode order")

    def append(self, layer: int) -> None:
        self._live.check(layer)
        c = self.calls[layer]
        rc = c.append_fn(*c.append_args)
        if rc:
            _lib.check(rc, f"append layer {layer}")

    def attend(self, layer: int, shared_blocks: bool | None = None) -> None:
        self._live.check(layer)
        c = self.calls[layer]
        fn = self.lib.wkv_paged_decode_gqa_grouped if self.grouped else self.lib.wkv_paged_decode_gqa
        rc = fn(*c.decode_args[c.shared_default if shared_blocks is None else bool(shared_blocks)])
        if rc:
            _lib.check(rc, f"decode layer {layer}")

    def step_layer(self, layer: int, shared_blocks: bool | None = None) -> None:
        """Append + attention of one layer in a single launch (plus the partition merge)."""
        self._live.check(layer)
        c = self.calls[layer]
        fn = self.lib.wkv_paged_decode_gqa_grouped if self.grouped else self.lib.wkv_append_paged_decode_gqa
        rc = fn(*c.fused_args[c.shared_default if shared_blocks is None else bool(shared_blocks)])
        if rc:
            _lib.check(rc, f"append+decode layer {layer}")

    def run(self, fused: bool = True, shared_blocks: bool | None = None) -> None:
        """One decode step over every layer (fused append + attention by default), with
        the step's read policy ``shared_blocks`` (None = each cache's default)."""
        self.prepare()
        for layer in range(len(self.calls)):
            if fused:
                self.step_layer(layer, shared_blocks)
            else:
                self.append(layer)
                self.attend(layer, shared_blocks)


class GraphDecodeStep:
    """A decode step captured once in a HIP graph and replayed every step.

    The engine runs its decode steps as captured graphs unless told otherwise
    (``enforce_eager`` defaults to False: wavelet/configs/config.py:1017, passed to
    the engine at wavelet/inference/engine.py:800). This records the whole step of a
    ``DecodeStep`` -- the dispatch-order launch and every layer's fused append +
    attention (+ partition merge) -- into one ``torch.cuda.CUDAGraph``, through the
    allocation-free entry point (``wkv_append_paged_decode_gqa_noalloc``: split-K
    partials in the library's static per-GPU scratch, so nothing is allocated and no
    memset is recorded); ``replay()`` is one graph launch on the current stream.

    The plan's buffers (q, key, value, out, block table, lengths, slots) are the
    graph's: refill them in place between steps, as for ``DecodeStep``. Its geometry
    is fixed at capture (batch, ``max_seq_len`` as an upper bound of every length the
    replays will see, partition, read policy ``shared_blocks``: None = each cache's
    default). Every call on a GPU shares that GPU's scratch: two plans' replays must
    not overlap (one stream, or ordered). Geometries whose partials exceed the scratch
    (``wkv_decode_workspace_size`` > ``WKV_NOALLOC_SCRATCH_BYTES``) are refused. The
    group-aware decode is not captured here.
    """

    def __init__(self, step: DecodeStep, *, shared_blocks: bool | None = None) -> None:
        if step.grouped:
            raise NotImplementedError("GraphDecodeStep captures the plain decode (no group-aware plan)")
        self.step = step
        caches, q, key, value, out = step._keep
        lib = step.lib
        batch = step.seq_lens.shape[0]
        # the launch's partition, waves per workgroup and chunks: partials (and the scratch)
        # only when a context spans more than one workgroup
        c0 = caches[0]
        bt_width = step.block_table.shape[1]
        part, waves, chunks = decode_plan(batch, c0.num_kv_heads, min(step.max_seq_len, bt_width * c0.block_size),
                                          c0.block_size, step.partition_size)
        need = lib.wkv_decode_workspace_size(batch, q[0].shape[1], c0.head_dim,
                                             min(step.max_seq_len, bt_width * c0.block_size), part * waves)
        if chunks > 1 and (need < 0 or need > _lib.WKV_NOALLOC_SCRATCH_BYTES):
            raise ValueError(f"the step's split-K partials need {need} bytes, beyond the "
                             f"{_lib.WKV_NOALLOC_SCRATCH_BYTES}-byte scratch of the allocation-free decode")
        dev = caches[0].device
        self._live = step._live
        self._live.check_all()
        order_ptr = step.order.data_ptr() if step.ordered else None
        bt, sl, slots = step.block_table, step.seq_lens, step.slot_mapping

        def calls(stream: int) -> list[tuple]:
            out_calls = []
            for layer, cache in enumerate(caches):
                qq, kk, vv, oo = q[layer], key[layer], value[layer], out[layer]
                out_calls.append((ctypes.byref(cache.descriptor(shared_blocks)), kk.data_ptr(), kk.stride(0),
                                  kk.stride(1), vv.data_ptr(), vv.stride(0), vv.stride(1), slots.data_ptr(),
                                  qq.data_ptr(), qq.stride(0), qq.stride(1), oo.data_ptr(), qq.shape[1],
                                  bt.data_ptr(), bt.stride(0), bt.shape[1], sl.data_ptr(), batch,
                                  step.max_seq_len, ctypes.c_float(step.scale), step.partition_size, order_ptr,
                                  stream))
            return out_calls

        fn = lib.wkv_append_paged_decode_gqa_noalloc
        # the scratch's address is looked up once per device, outside the capture (a
        # zero-length call validates the arguments and launches nothing)
        first = calls(torch.cuda.current_stream(dev).cuda_stream)[0]
        _lib.check(fn(*first[:17], 0, *first[18:]), "allocation-free decode (set-up)")
        self.graph = torch.cuda.CUDAGraph()
        capture = torch.cuda.Stream(dev)
        capture.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.graph(self.graph, stream=capture):
            cur = torch.cuda.current_stream(dev).cuda_stream
            if step.ordered:
                _lib.check(lib.wkv_decode_order(sl.data_ptr(), batch, step.order.data_ptr(), cur), "decode order")
            for layer, args in enumerate(calls(cur)):
                _lib.check(fn(*args), f"allocation-free append+decode layer {layer}")
        torch.cuda.current_stream(dev).wait_stream(capture)

    def replay(self) -> None:
        """One decode step over every layer: one graph launch."""
        self._live.check_all()
        self.graph.replay()


class MLADecodeStep:
    """Pre-validated MLA decode for every layer: append one latent entry per
    sequence, then weight-absorbed attention over the latent cache."""

    def __init__(self, caches, q_nope: list[torch.Tensor], q_pe: list[torch.Tensor], kv_c: list[torch.Tensor],
                 k_pe: list[torch.Tensor], out: list[torch.Tensor], block_table: torch.Tensor, seq_lens: torch.Tensor,
                 slot_mapping: torch.Tensor, scale: float, max_seq_len: int, partition_size: int = 0) -> None:
        if not caches:
            raise ValueError("no layers")
        c0 = caches[0]
        dev = c0.device
        self.block_table, self.seq_lens = check_tables(block_table, seq_lens, dev, c0.block_size, strict=True)
        batch = self.seq_lens.shape[0]
        slot_mapping = _plan_slots(slot_mapping, dev, batch)
        if not len(q_nope) == len(q_pe) == len(kv_c) == len(k_pe) == len(out) == len(caches):
            raise ValueError("q_nope, q_pe, kv_c, k_pe and out need one tensor per layer")
        self._live = _Live(caches)
        heads = q_nope[0].shape[1]
        lib = _lib.load()
        need = lib.wkv_mla_workspace_size(batch, heads, c0.kv_lora_rank, max_seq_len, int(partition_size))
        if need < 0:
            raise ValueError("invalid MLA decode geometry")
        self.workspace = _workspace(dev, need)
        self.stream = torch.cuda.current_stream(dev).cuda_stream
        self.lib = lib
        self.calls = []
        for layer, cache in enumerate(caches):
            qn, qp, kc, kp, oo = q_nope[layer], q_pe[layer], kv_c[layer], k_pe[layer], out[layer]
            for name, t, shape in (("q_nope", qn, (batch, heads, cache.kv_lora_rank)),
                                   ("q_pe", qp, (batch, heads, cache.rope_dim)),
                                   ("out", oo, (batch, heads, cache.kv_lora_rank)),
                                   ("kv_c", kc, (slot_mapping.numel(), cache.kv_lora_rank)),
                                   ("k_pe", kp, (slot_mapping.numel(), cache.rope_dim))):
                if t.dtype != torch.bfloat16 or tuple(t.shape) != shape or not t.is_contiguous() or t.device != dev:
                    raise ValueError(f"layer {layer}: {name} must be a contiguous bfloat16 {shape} tensor on {dev}")
            desc = ctypes.byref(cache.descriptor())
            append_args = (desc, kc.data_ptr(), kc.stride(0), kp.data_ptr(), kp.stride(0), slot_mapping.data_ptr(),
                           slot_mapping.numel(), self.stream)
            decode_args = (desc, qn.data_ptr(), qn.stride(0), qn.stride(1), qp.data_ptr(), qp.stride(0), qp.stride(1),
                           oo.data_ptr(), heads, self.block_table.data_ptr(), self.block_table.stride(0),
                           self.block_table.shape[1], self.seq_lens.data_ptr(), batch, int(max_seq_len),
                           ctypes.c_float(scale), int(partition_size), self.workspace.data_ptr(),
                           self.workspace.numel(), self.stream)
            fused_args = (desc, kc.data_ptr(), kc.stride(0), kp.data_ptr(), kp.stride(0), slot_mapping.data_ptr(),
                          *decode_args[1:])
            self.calls.append((append_args, decode_args, fused_args))
        self._keep = (caches, q_nope, q_pe, kv_c, k_pe, out, slot_mapping)

    def append(self, layer: int) -> None:
        self._live.check(layer)
        rc = self.lib.wkv_mla_append(*self.calls[layer][0])
        if rc:
            _lib.check(rc, f"mla append layer {layer}")

    def attend(self, layer: int) -> None:
        self._live.check(layer)
        rc = self.lib.wkv_paged_decode_mla(*self.calls[layer][1])
        if rc:
            _lib.check(rc, f"mla decode layer {layer}")

    def step_layer(self, layer: int) -> None:
        """Latent append + attention of one layer in a single launch (plus the partition merge)."""
        self._live.check(layer)
        rc = self.lib.wkv_append_paged_decode_mla(*self.calls[layer][2])
        if rc:
            _lib.check(rc, f"mla append+decode layer {layer}")

    def run(self) -> None:
        for layer in range(len(self.calls)):
            self.step_layer(layer)


class PrefillStep:
    """Pre-validated prompt step for every layer: append the new tokens' K/V and
    attend causally over each sequence's paged context (``prefill_gqa``).

    ``q[l]`` ``[T, Hq, D]``, ``key[l]`` / ``value[l]`` ``[T, Hkv, D]`` and
    ``out[l]`` are layer ``l``'s buffers; ``cu_seqlens_q [B+1]`` int32 splits
    the ``T`` rows by sequence and ``slot_mapping [T]`` places them.
    """

    def __init__(self, caches: list[PagedKVCache], q: list[torch.Tensor], key: list[torch.Tensor],
                 value: list[torch.Tensor], out: list[torch.Tensor], block_table: torch.Tensor,
                 seq_lens: torch.Tensor, cu_seqlens_q: torch.Tensor, slot_mapping: torch.Tensor, scale: float,
                 max_query_len: int, max_seq_len: int) -> None:
        if not caches:
            raise ValueError("no layers")
        dev = caches[0].device
        self.block_table, self.seq_lens = check_tables(block_table, seq_lens, dev, caches[0].block_size,
                                                       strict=True)
        batch = self.seq_lens.shape[0]
        _require_cuda(cu_seqlens_q, "cu_seqlens_q", dev)
        if (cu_seqlens_q.dtype != torch.int32 or tuple(cu_seqlens_q.shape) != (batch + 1,)
                or not cu_seqlens_q.is_contiguous() or cu_seqlens_q.device != dev):
            raise ValueError(f"cu_seqlens_q must be a contiguous int32 [{batch + 1}] tensor on {dev}")
        slot_mapping = _plan_slots(slot_mapping, dev, None)
        if not len(q) == len(key) == len(value) == len(out) == len(caches):
            raise ValueError("q, key, value and out need one tensor per layer")
        self._live = _Live(caches)
        T = slot_mapping.numel()
        self.lib = lib = _lib.load()
        self.stream = torch.cuda.current_stream(dev).cuda_stream
        self.calls = []
        for layer, cache in enumerate(caches):
            qq, kk, vv, oo = q[layer], key[layer], value[layer], out[layer]
            hq = qq.shape[1]
            for name, t, shape in (("q", qq, (T, hq, cache.head_dim)), ("out", oo, (T, hq, cache.head_dim)),
                                   ("key", kk, (T, cache.num_kv_heads, cache.head_dim)),
                                   ("value", vv, (T, cache.num_kv_heads, cache.head_dim))):
                if t.dtype != torch.bfloat16 or tuple(t.shape) != shape or not t.is_contiguous() or t.device != dev:
                    raise ValueError(f"layer {layer}: {name} must be a contiguous bfloat16 {shape} tensor on {dev}")
            desc = ctypes.byref(cache.descriptor())
            kv = (kk.data_ptr(), kk.stride(0), kk.stride(1), vv.data_ptr(), vv.stride(0), vv.stride(1),
                  slot_mapping.data_ptr())
            tail = (qq.data_ptr(), qq.stride(0), qq.stride(1), oo.data_ptr(), oo.stride(0), oo.stride(1), hq,
                    cu_seqlens_q.data_ptr(), self.seq_lens.data_ptr(), self.block_table.data_ptr(),
                    self.block_table.stride(0), self.block_table.shape[1], batch, int(max_query_len),
                    int(max_seq_len), ctypes.c_float(scale), self.stream)
            fn = lib.wkv_append_fp8 if cache.kv_dtype == "fp8_e4m3" else lib.wkv_append
            self.calls.append((fn, (desc, *kv, T, self.stream), (desc, *kv, T, *tail),
                               (desc, None, 0, 0, None, 0, 0, None, 0, *tail)))
        self._keep = (caches, q, key, value, out, cu_seqlens_q, slot_mapping)

    def append(self, layer: int) -> None:
        self._live.check(layer)
        fn, args, _, _ = self.calls[layer]
        rc = fn(*args)
        if rc:
            _lib.check(rc, f"append layer {layer}")

    def attend(self, layer: int) -> None:
        self._live.check(layer)
        rc = self.lib.wkv_prefill_gqa(*self.calls[layer][3])
        if rc:
            _lib.check(rc, f"prefill layer {layer}")

    def step_layer(self, layer: int) -> None:
        """Append + causal attention of one layer (two launches: the append, then the attention)."""
        self._live.check(layer)
        rc = self.lib.wkv_prefill_gqa(*self.calls[layer][2])
        if rc:
            _lib.check(rc, f"append+prefill layer {layer}")

    def run(self) -> None:
        for layer in range(len(self.calls)):
            self.step_layer(layer)
