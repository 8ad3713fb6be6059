"""Paged KV caches on the GPU: the cache half of the engine's KV surface.

The reference sizes one KV pool per layer inside the vLLM engine it builds
(wavelet/inference/engine.py:776-825; ``gpu_memory_utilization``,
``max_model_len``, KV dtype = model dtype) and appends every new token of a
decode step through a slot mapping before attention (``llm.generate``,
engine.py:887; HF analogue ``past_key_values.update`` at
wavelet/kernels/patch.py:173-180). ``PagedKVCache`` is one such layer; the
heavy lifting is done by libwkv.so through its C ABI, and PyTorch only owns
the memory.

Physical layout (x = 16 // element bytes)::

    k  [num_blocks, num_kv_heads, head_dim // x, block_size, x]
    v  [num_blocks, num_kv_heads, head_dim, block_size]
    k_scale, v_scale  [num_blocks, num_kv_heads] float32   (fp8 only)

The contiguous ``gather`` output ``[tokens, num_kv_heads, head_dim]`` is the
layout-independent contract.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

KV_DTYPES = {"bf16": _lib.WKV_KV_BF16, "fp8_e4m3": _lib.WKV_KV_FP8_E4M3}


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, cache is on {device}")


def _slots(slot_mapping: torch.Tensor, n: int, device: torch.device) -> torch.Tensor:
    _require_cuda(slot_mapping, "slot_mapping", device)
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or slot_mapping.numel() != n:
        raise ValueError(f"slot_mapping must be int64 [{n}] (got {slot_mapping.dtype} {tuple(slot_mapping.shape)})")
    return slot_mapping.contiguous()


def _token_rows(x: torch.Tensor, name: str, shape: tuple[int, ...], device: torch.device) -> torch.Tensor:
    _require_cuda(x, name, device)
    if x.dtype != torch.bfloat16 or tuple(x.shape[1:]) != shape:
        raise ValueError(f"{name} must be bfloat16 [T, {', '.join(map(str, shape))}] (got {x.dtype} {tuple(x.shape)})")
    if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:-1]) or x.data_ptr() % 16:
        x = x.contiguous()
    return x


class PagedKVCache:
    """One layer's paged K/V cache (bf16, or fp8-e4m3 with per-(block, head) scales)."""

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        kv_dtype: str = "bf16",
        device: torch.device | str | None = None,
        shared_blocks: bool = False,
    ) -> None:
        if kv_dtype not in KV_DTYPES:
            raise ValueError(f"kv_dtype must be one of {sorted(KV_DTYPES)} (got {kv_dtype!r})")
        if block_size <= 0 or block_size % 16:
            raise ValueError(f"block_size must be a positive multiple of 16 (got {block_size})")
        if head_dim not in (64, 128):
            raise NotImplementedError(f"head_dim {head_dim} not supported (64 or 128)")
        if num_blocks <= 0 or num_kv_heads <= 0:
            raise ValueError("num_blocks and num_kv_heads must be positive")
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self._shared_blocks = bool(shared_blocks)
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.kv_dtype = kv_dtype
        self._allocate()

    def _allocate(self) -> None:
        fp8 = self.kv_dtype == "fp8_e4m3"
        elem = torch.uint8 if fp8 else torch.bfloat16
        x = 16 if fp8 else 8
        nb, h, d, bs = self.num_blocks, self.num_kv_heads, self.head_dim, self.block_size
        self.k = torch.zeros((nb, h, d // x, bs, x), dtype=elem, device=self.device)
        self.v = torch.zeros((nb, h, d, bs), dtype=elem, device=self.device)
        self.k_scale = torch.zeros((nb, h), dtype=torch.float32, device=self.device) if fp8 else None
        self.v_scale = torch.zeros((nb, h), dtype=torch.float32, device=self.device) if fp8 else None
        # one descriptor per read policy (the flag is read per call); _desc is the default one
        self._descs = {
            shared: _lib.WkvCache(
                k=self.k.data_ptr(),
                v=self.v.data_ptr(),
                k_scale=self.k_scale.data_ptr() if fp8 else None,
                v_scale=self.v_scale.data_ptr() if fp8 else None,
                num_blocks=self.num_blocks,
                block_size=self.block_size,
                num_kv_heads=self.num_kv_heads,
                head_dim=self.head_dim,
                kv_dtype=KV_DTYPES[self.kv_dtype],
                flags=_lib.CACHE_SHARED_BLOCKS if shared else 0,
            )
            for shared in (False, True)
        }
        self._desc = self._descs[self._shared_blocks]

    # -- sleep / wake (the engine's sleep(level=1) / wake_up(tags=["kv_cache"]),
    #    wavelet/inference/engine.py:858-873) ---------------------------------
    @property
    def asleep(self) -> bool:
        return self._desc is None

    def sleep(self) -> None:
        """Release the pool's device memory; the contents are discarded."""
        self.k = self.v = self.k_scale = self.v_scale = None
        self._desc = None
        self._descs = None

    def wake_up(self) -> None:
        """Allocate the pool again (zeroed); a no-op when awake."""
        if self.asleep:
            self._allocate()

    # -- properties ---------------------------------------------------------
    @property
    def capacity_tokens(self) -> int:
        """``num_gpu_blocks * block_size`` (wavelet/orchestrator/inference_metrics.py:125-133)."""
        return self.num_blocks * self.block_size

    @property
    def nbytes(self) -> int:
        """Device bytes the pool holds while awake."""
        elem = 1 if self.kv_dtype == "fp8_e4m3" else 2
        n = 2 * self.num_blocks * self.num_kv_heads * self.head_dim * self.block_size * elem
        if self.kv_dtype == "fp8_e4m3":
            n += 2 * self.num_blocks * self.num_kv_heads * 4
        return n

    @property
    def shared_blocks(self) -> bool:
        """The decodes' default read policy (fixed at construction; a call can choose per
        step): True when several sequences may read one block (prefix caching, forks) --
        K/V reads then keep blocks cached for the next reader; False streams them past the
        caches as read-once data (3-9% faster when nothing is shared)."""
        return self._shared_blocks

    def descriptor(self, shared_blocks: bool | None = None) -> ctypes.Structure:
        """The C descriptor of this cache, with the read policy ``shared_blocks`` (None =
        the cache's default)."""
        if self._desc is None:
            raise RuntimeError("the KV cache is asleep: call wake_up() first")
        return self._desc if shared_blocks is None else self._descs[bool(shared_blocks)]

    # -- operations ---------------------------------------------------------
    def append(self, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Write ``key[t], value[t]`` ([T, Hkv, D] bf16) at ``slot_mapping[t]`` (-1 = skip).

        fp8 caches quantise on the way in; see ``wkv_append_fp8`` for the
        per-(block, head) scale rule.
        """
        shape = (self.num_kv_heads, self.head_dim)
        key = _token_rows(key, "key", shape, self.device)
        value = _token_rows(value, "value", shape, self.device)
        if key.shape[0] != value.shape[0]:
            raise ValueError("key and value must have the same number of tokens")
        n = key.shape[0]
        slots = _slots(slot_mapping, n, self.device)
        lib = _lib.load()
        fn = lib.wkv_append_fp8 if self.kv_dtype == "fp8_e4m3" else lib.wkv_append
        rc = fn(
            ctypes.byref(self.descriptor()),
            key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            slots.data_ptr(), n, _stream(self.device),
        )
        _lib.check(rc, "append")

    def gather(
        self,
        block_table: torch.Tensor,
        seq_lens: torch.Tensor,
        *,
        dequant: bool = False,
        total_tokens: int | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous ``[sum(seq_lens), Hkv, D]`` copies of every sequence's K and V.

        ``dequant`` turns fp8 codes into bf16 values (exact); otherwise the raw
        stored elements come back (bf16, or uint8 fp8 codes).
        """
        block_table, seq_lens = check_tables(block_table, seq_lens, self.device, self.block_size)
        batch = seq_lens.shape[0]
        cu = torch.zeros(batch, dtype=torch.int64, device=self.device)
        if batch > 1:
            cu[1:] = torch.cumsum(seq_lens[:-1].to(torch.int64), 0)
        total = int(seq_lens.to(torch.int64).sum().item()) if total_tokens is None else int(total_tokens)
        fp8 = self.kv_dtype == "fp8_e4m3"
        if dequant and not fp8:
            raise ValueError("dequant applies to fp8 caches only")
        dt = torch.bfloat16 if (dequant or not fp8) else torch.uint8
        shape = (total, self.num_kv_heads, self.head_dim)
        out_k = torch.empty(shape, dtype=dt, device=self.device)
        out_v = torch.empty(shape, dtype=dt, device=self.device)
        if total == 0 or batch == 0:
            return out_k, out_v
        rc = _lib.load().wkv_gather(
            ctypes.byref(self.descriptor()),
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            seq_lens.data_ptr(), cu.data_ptr(), batch,
            out_k.data_ptr(), out_v.data_ptr(), int(dequant), _stream(self.device),
        )
        _lib.check(rc, "gather")
        return out_k, out_v

    def copy_blocks(self, block_mapping: torch.Tensor) -> None:
        """Copy block ``mapping[i, 0]`` onto ``mapping[i, 1]`` (K, V and scales)."""
        _require_cuda(block_mapping, "block_mapping", self.device)
        if block_mapping.dtype != torch.int64 or block_mapping.dim() != 2 or block_mapping.shape[1] != 2:
            raise ValueError("block_mapping must be int64 [n, 2]")
        m = block_mapping.contiguous()
        rc = _lib.load().wkv_copy_blocks(ctypes.byref(self.descriptor()), m.data_ptr(), m.shape[0], _stream(self.device))
        _lib.check(rc, "copy_blocks")


class MLALatentCache:
    """One layer's MLA latent cache ``[num_blocks, block_size, kv_lora_rank + rope_dim]`` bf16."""

    def __init__(self, num_blocks: int, block_size: int = 64, kv_lora_rank: int = 512, rope_dim: int = 64,
                 device: torch.device | str | None = None) -> None:
        if block_size <= 0 or block_size % 16:
            raise ValueError(f"block_size must be a positive multiple of 16 (got {block_size})")
        if kv_lora_rank % 8 or rope_dim % 8:
            raise ValueError("kv_lora_rank and rope_dim must be multiples of 8")
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self.kv_lora_rank = int(kv_lora_rank)
        self.rope_dim = int(rope_dim)
        self._allocate()

    def _allocate(self) -> None:
        self.latent = torch.zeros((self.num_blocks, self.block_size, self.kv_lora_rank + self.rope_dim),
                                  dtype=torch.bfloat16, device=self.device)
        self._desc = _lib.WkvMlaCache(
            latent=self.latent.data_ptr(),
            num_blocks=self.num_blocks,
            block_size=self.block_size,
            kv_lora_rank=self.kv_lora_rank,
            rope_dim=self.rope_dim,
        )

    @property
    def asleep(self) -> bool:
        return self._desc is None

    def sleep(self) -> None:
        """Release the latent pool's device memory; the contents are discarded."""
        self.latent = None
        self._desc = None

    def wake_up(self) -> None:
        """Allocate the latent pool again (zeroed); a no-op when awake."""
        if self.asleep:
            self._allocate()

    @property
    def capacity_tokens(self) -> int:
        return self.num_blocks * self.block_size

    @property
    def nbytes(self) -> int:
        return self.num_blocks * self.block_size * (self.kv_lora_rank + self.rope_dim) * 2

    def descriptor(self) -> ctypes.Structure:
        if self._desc is None:
            raise RuntimeError("the KV cache is asleep: call wake_up() first")
        return self._desc

    def append(self, kv_c: torch.Tensor, k_pe: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """``latent[slot[t]] = concat(kv_c[t], k_pe[t])`` (vLLM's concat_and_cache_mla)."""
        for name, x, w in (("kv_c", kv_c, self.kv_lora_rank), ("k_pe", k_pe, self.rope_dim)):
            _require_cuda(x, name, self.device)
            if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != w:
                raise ValueError(f"{name} must be bfloat16 [T, {w}]")
        if kv_c.shape[0] != k_pe.shape[0]:
            raise ValueError("kv_c and k_pe must have the same number of tokens")
        if kv_c.stride(1) != 1 or kv_c.stride(0) % 8 or kv_c.data_ptr() % 16:
            kv_c = kv_c.contiguous()
        if k_pe.stride(1) != 1 or k_pe.stride(0) % 8 or k_pe.data_ptr() % 16:
            k_pe = k_pe.contiguous()
        n = kv_c.shape[0]
        slots = _slots(slot_mapping, n, self.device)
        rc = _lib.load().wkv_mla_append(
            ctypes.byref(self.descriptor()), kv_c.data_ptr(), kv_c.stride(0), k_pe.data_ptr(), k_pe.stride(0),
            slots.data_ptr(), n, _stream(self.device),
        )
        _lib.check(rc, "mla_append")

    def gather(self, block_table: torch.Tensor, seq_lens: torch.Tensor, *,
               total_tokens: int | None = None) -> torch.Tensor:
        """Contiguous ``[sum(seq_lens), kv_lora_rank + rope_dim]`` bf16 copy of every
        sequence's latent rows (``c_kv`` then ``k_pe``), in sequence order: the
        cached-context read of an MLA chunked prefill or prefix-cache hit."""
        block_table, seq_lens = check_tables(block_table, seq_lens, self.device, self.block_size)
        batch = seq_lens.shape[0]
        cu = torch.zeros(batch, dtype=torch.int64, device=self.device)
        if batch > 1:
            cu[1:] = torch.cumsum(seq_lens[:-1].to(torch.int64), 0)
        total = int(seq_lens.to(torch.int64).sum().item()) if total_tokens is None else int(total_tokens)
        out = torch.empty((total, self.kv_lora_rank + self.rope_dim), dtype=torch.bfloat16, device=self.device)
        if total == 0 or batch == 0:
            return out
        rc = _lib.load().wkv_mla_gather(
            ctypes.byref(self.descriptor()), block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            seq_lens.data_ptr(), cu.data_ptr(), batch, out.data_ptr(), _stream(self.device),
        )
        _lib.check(rc, "mla_gather")
        return out

    def copy_blocks(self, block_mapping: torch.Tensor) -> None:
        """Copy latent block ``mapping[i, 0]`` onto ``mapping[i, 1]`` (copy-on-write)."""
        _require_cuda(block_mapping, "block_mapping", self.device)
        if block_mapping.dtype != torch.int64 or block_mapping.dim() != 2 or block_mapping.shape[1] != 2:
            raise ValueError("block_mapping must be int64 [n, 2]")
        m = block_mapping.contiguous()
        rc = _lib.load().wkv_mla_copy_blocks(ctypes.byref(self.descriptor()), m.data_ptr(), m.shape[0],
                                             _stream(self.device))
        _lib.check(rc, "mla_copy_blocks")


def check_tables(block_table: torch.Tensor, seq_lens: torch.Tensor, device: torch.device,
                 block_size: int, *, strict: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Validate ``block_table [B, M] int32`` and ``seq_lens [B] int32`` (device tensors).

    A one-shot call may hand in a block table whose rows are not contiguous or
    a strided ``seq_lens``: those are copied. ``strict`` (the pre-validated
    plans, which keep the caller's tensors and expect them refilled in place)
    refuses them instead, since a copy would never see the caller's updates.
    """
    _require_cuda(block_table, "block_table", device)
    _require_cuda(seq_lens, "seq_lens", device)
    if block_table.dtype != torch.int32 or block_table.dim() != 2:
        raise ValueError(f"block_table must be int32 [B, max_blocks] (got {block_table.dtype} {tuple(block_table.shape)})")
    if seq_lens.dtype != torch.int32 or seq_lens.dim() != 1 or seq_lens.shape[0] != block_table.shape[0]:
        raise ValueError("seq_lens must be int32 [B] matching block_table")
    if strict:
        if block_table.stride(1) != 1 or not seq_lens.is_contiguous():
            raise ValueError("a plan needs a block_table with contiguous rows (stride(1) == 1) and a contiguous "
                             "seq_lens: it reads the tensors handed to it on every step")
        return block_table, seq_lens
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    return block_table, seq_lens.contiguous()


def validate_tables(block_table: torch.Tensor, seq_lens: torch.Tensor, num_blocks: int, block_size: int) -> None:
    """Debug check (synchronises): every block-table entry a sequence reads is a real block.

    The kernels never fault on a bad id (they treat it as masked slots); this
    turns such a table into a ValueError instead.
    """
    m = block_table.shape[1]
    if int(seq_lens.max().item() if seq_lens.numel() else 0) > m * block_size:
        raise ValueError("a sequence is longer than its block table")
    used = (torch.arange(m, device=block_table.device)[None, :] * block_size) < seq_lens[:, None].to(torch.int64)
    ids = block_table[used]
    if ids.numel() and (int(ids.min().item()) < 0 or int(ids.max().item()) >= num_blocks):
        raise ValueError(f"block table references a block outside [0, {num_blocks})")


def validate_group_prefix(block_table, seq_lens, prefix_lens, group_size: int, block_size: int, *,
                          appending: bool = False) -> None:
    """Debug check (synchronises) of a group-aware decode's ``prefix_lens`` claim.

    The claim: group ``g``'s first ``n_g`` blocks are the same physical blocks in
    every member's table, ``n_g = min(prefix_lens[g], shortest member context
    (minus the token a fused append adds)) // block_size``.
    ``paged_decode_gqa_grouped`` reads every member through its own table, so a
    wrong claim cannot change its result; it reads the claimed tokens with the
    cached policy, so a claim that covers private blocks only wastes cache
    capacity on them. This raises ValueError naming the first (group, member,
    block) that breaks the claim. Accepts torch tensors (any device) or numpy
    arrays.
    """
    import numpy as np

    def host(x):
        return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)

    bt, lens, pre = host(block_table), host(seq_lens).astype(np.int64), host(prefix_lens).astype(np.int64)
    group_size = int(group_size)
    if bt.ndim != 2 or lens.shape != (bt.shape[0],):
        raise ValueError("block_table must be [B, max_blocks] and seq_lens [B]")
    batch = bt.shape[0]
    if group_size < 1:
        raise ValueError(f"group_size must be positive (got {group_size})")
    n_groups = -(-batch // group_size)
    if pre.shape != (n_groups,):
        raise ValueError(f"prefix_lens must have one entry per group ({n_groups})")
    if (pre < 0).any():
        raise ValueError("prefix_lens must be non-negative")
    for g in range(n_groups):
        b0, b1 = g * group_size, min((g + 1) * group_size, batch)
        shortest = int(lens[b0:b1].min()) - (1 if appending else 0)
        n = max(min(int(pre[g]), shortest), 0) // int(block_size)
        n = min(n, bt.shape[1])
        if n == 0:
            continue
        lead = bt[b0, :n]
        for b in range(b0 + 1, b1):
            diff = np.nonzero(bt[b, :n] != lead)[0]
            if diff.size:
                j = int(diff[0])
                raise ValueError(f"group {g}: prefix_lens {int(pre[g])} claims block {j} shared, but member {b} "
                                 f"holds block {int(bt[b, j])} where member {b0} holds {int(lead[j])}")
