"""Host-side block management for the paged KV cache.

The reference leaves block allocation, prefix sharing and prefix-cache keying
to the engine it drives; what it relies on is visible at its call sites:

* GRPO groups: ``SamplingParams(n=num_generations)`` (wavelet/inference/
  engine.py:69-90) -- the ``n`` members of a group share the prompt's KV;
* ``cache_salt`` (engine.py:1034-1038, :500-501): prefix-cache blocks are keyed
  by salt, so requests of different policy steps never share cached KV;
* ``reset_prefix_cache`` after an adapter reload and before sleep
  (engine.py:858-869, :1236-1242);
* KV capacity ``num_gpu_blocks * block_size`` and usage, scraped as
  ``vllm:cache_config_info`` / ``vllm:kv_cache_usage_perc``
  (wavelet/orchestrator/inference_metrics.py:16-20, :125-133).

``BlockManager`` provides those semantics for ``PagedKVCache`` block tables:
ref-counted physical blocks, prompt sharing across a group (``fork`` /
``share_prefix``), copy-on-write of a shared partially filled block (the caller
applies the returned pairs with ``PagedKVCache.copy_blocks``), a salt-keyed
index of full prompt blocks, and the Prometheus lines the reference parses.
It is pure Python bookkeeping: one manager serves every layer's cache, since
all layers share one block table per sequence.
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict, deque
from dataclasses import dataclass, field

import numpy as np


@dataclass
class _Seq:
    blocks: list[int] = field(default_factory=list)
    length: int = 0


class BlockManager:
    """Allocates physical KV blocks to sequences; one table per sequence."""

    def __init__(self, num_blocks: int, block_size: int, *, enable_prefix_caching: bool = True,
                 max_model_len: int | None = None) -> None:
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        if max_model_len is not None and int(max_model_len) <= 0:
            raise ValueError(f"max_model_len must be positive (got {max_model_len})")
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self.enable_prefix_caching = enable_prefix_caching
        # the engine's context limit (RLVLLMConfig.max_model_len, configs/config.py:1005-1009): no sequence
        # grows past it, and block tables are this many blocks wide
        self.max_model_len = None if max_model_len is None else int(max_model_len)
        self._free: deque[int] = deque(range(self.num_blocks))
        self._ref = np.zeros(self.num_blocks, dtype=np.int64)
        self._seqs: dict[object, _Seq] = {}
        self._index: dict[bytes, int] = {}  # full-block chain hash -> block id
        self._hash_of: dict[int, bytes] = {}  # block id -> its chain hash (indexed blocks)
        self._evictable: OrderedDict[int, None] = OrderedDict()  # indexed blocks with ref 0, LRU first

    # -- capacity and metrics --------------------------------------------------
    @property
    def max_blocks_per_seq(self) -> int | None:
        """Block-table width that ``max_model_len`` implies (None without a limit)."""
        if self.max_model_len is None:
            return None
        return -(-self.max_model_len // self.block_size)

    @property
    def capacity_tokens(self) -> int:
        """``num_gpu_blocks * block_size`` (inference_metrics.py:125-133)."""
        return self.num_blocks * self.block_size

    @property
    def num_free_blocks(self) -> int:
        return len(self._free) + len(self._evictable)

    @property
    def usage(self) -> float:
        """Fraction of blocks held by live sequences (``vllm:kv_cache_usage_perc``)."""
        return 1.0 - self.num_free_blocks / self.num_blocks

    def metrics_text(self) -> str:
        """The Prometheus lines the reference's scraper reads for KV usage and capacity."""
        return (
            f"vllm:kv_cache_usage_perc {self.usage:.6f}\n"
            f'vllm:cache_config_info{{block_size="{self.block_size}",num_gpu_blocks="{self.num_blocks}"}} 1\n'
        )

    # -- allocation ------------------------------------------------------------
    def _take(self) -> int:
        if self._free:
            b = self._free.popleft()
        elif self._evictable:
            b, _ = self._evictable.popitem(last=False)  # least recently released cached block
            self._index.pop(self._hash_of.pop(b), None)
        else:
            raise MemoryError("out of KV cache blocks")
        self._ref[b] = 1
        return b

    def _release(self, b: int) -> None:
        self._ref[b] -= 1
        if self._ref[b] == 0:
            if b in self._hash_of:
                self._evictable[b] = None  # stays matchable until evicted or reset
            else:
                self._free.append(b)

    def _chain(self, prev: bytes, salt: str | None, tokens) -> bytes:
        h = hashlib.sha256(prev)
        h.update(b"\x00" if salt is None else b"\x01" + str(salt).encode())
        h.update(np.asarray(tokens, dtype=np.int64).tobytes())
        return h.digest()

    def allocate(self, seq_id, prompt_tokens, *, cache_salt: str | None = None) -> int:
        """Blocks for a new sequence's prompt; returns how many leading tokens are already cached.

        Full prompt blocks are looked up in the prefix index by a hash chain
        over (salt, token ids); matches are shared (ref-counted) instead of
        recomputed, so the caller only writes tokens from the returned count on.
        """
        if seq_id in self._seqs:
            raise ValueError(f"sequence {seq_id!r} already allocated")
        tokens = np.asarray(prompt_tokens, dtype=np.int64)
        if self.max_model_len is not None and len(tokens) > self.max_model_len:
            raise ValueError(f"prompt of {len(tokens)} tokens is longer than max_model_len {self.max_model_len}")
        bs = self.block_size
        n_full = len(tokens) // bs
        seq = _Seq()
        prev = b""
        reused = 0
        hashes = []
        for i in range(n_full):
            prev = self._chain(prev, cache_salt, tokens[i * bs:(i + 1) * bs])
            hashes.append(prev)
        if self.enable_prefix_caching:
            for h in hashes:
                b = self._index.get(h)
                if b is None:
                    break
                if self._ref[b] == 0:
                    self._evictable.pop(b, None)
                self._ref[b] += 1
                seq.blocks.append(b)
                reused += bs
        try:
            while len(seq.blocks) * bs < len(tokens):
                seq.blocks.append(self._take())
        except MemoryError:
            for b in seq.blocks:
                self._release(b)
            raise
        if self.enable_prefix_caching:
            for i in range(reused // bs, n_full):
                b = seq.blocks[i]
                if hashes[i] not in self._index:
                    self._index[hashes[i]] = b
                    self._hash_of[b] = hashes[i]
        seq.length = len(tokens)
        self._seqs[seq_id] = seq
        return reused

    def fork(self, parent, child) -> None:
        """``child`` shares every block of ``parent`` (n > 1 sampling of one prompt)."""
        self.share_prefix(parent, [child], None)

    def share_prefix(self, src_seq, dst_seqs, n_blocks: int | None) -> None:
        """New sequences ``dst_seqs`` start with ``src_seq``'s first ``n_blocks`` blocks (all if None)."""
        src = self._seqs[src_seq]
        n = len(src.blocks) if n_blocks is None else int(n_blocks)
        if n > len(src.blocks):
            raise ValueError(f"{src_seq!r} has only {len(src.blocks)} blocks")
        length = src.length if n_blocks is None else min(src.length, n * self.block_size)
        for dst in dst_seqs:
            if dst in self._seqs:
                raise ValueError(f"sequence {dst!r} already allocated")
            for b in src.blocks[:n]:
                self._ref[b] += 1
            self._seqs[dst] = _Seq(blocks=list(src.blocks[:n]), length=length)

    def _append_plan(self, seq_ids, num_tokens: int) -> int:
        """New blocks ``append_slots(seq_ids, num_tokens)`` would take (fresh blocks and
        copy-on-write copies), counted without changing any state; raises ValueError for a
        sequence listed twice or one that would pass ``max_model_len``."""
        if num_tokens < 0:
            raise ValueError(f"num_tokens must be non-negative (got {num_tokens})")
        if len(set(seq_ids)) != len(seq_ids):
            raise ValueError("a sequence is listed twice")
        bs = self.block_size
        released: dict[int, int] = {}  # block -> references the plan has already moved off it
        need = 0
        for sid in seq_ids:
            seq = self._seqs[sid]
            if self.max_model_len is not None and seq.length + num_tokens > self.max_model_len:
                raise ValueError(f"sequence {sid!r} at {seq.length} tokens cannot take {num_tokens} more: "
                                 f"max_model_len is {self.max_model_len}")
            if num_tokens == 0:
                continue
            pos = seq.length
            if pos < len(seq.blocks) * bs:  # the first token lands in an existing, partly filled block
                last = seq.blocks[pos // bs]
                if self._ref[last] - released.get(last, 0) > 1:
                    need += 1
                    released[last] = released.get(last, 0) + 1
            need += max(-(-(pos + num_tokens) // bs) - len(seq.blocks), 0)
        return need

    def append_slots(self, seq_ids, num_tokens: int = 1) -> tuple[np.ndarray, list[tuple[int, int]]]:
        """Reserve ``num_tokens`` new token slots per sequence (a decode step: one).

        Returns the int64 slots, sequence-major (``[len(seq_ids) * num_tokens]``:
        sequence ``i``'s tokens at ``i * num_tokens ..``), and the copy-on-write
        pairs ``(src_block, dst_block)`` to apply with ``copy_blocks`` on every
        layer (``KVPool.copy_blocks``) *before* the append: a sequence about to
        write into a block it still shares gets a private copy first. Nothing
        changes unless every sequence can take its tokens: one that would pass
        ``max_model_len`` raises ValueError, and a step needing more blocks than
        are free raises MemoryError, before any state moves.
        """
        seq_ids = list(seq_ids)
        need = self._append_plan(seq_ids, int(num_tokens))
        if need > self.num_free_blocks:
            raise MemoryError(f"out of KV cache blocks: the step needs {need}, {self.num_free_blocks} are free")
        slots = np.empty(len(seq_ids) * num_tokens, dtype=np.int64)
        cow: list[tuple[int, int]] = []
        bs = self.block_size
        for i, sid in enumerate(seq_ids):
            seq = self._seqs[sid]
            for t in range(num_tokens):
                pos = seq.length
                if pos == len(seq.blocks) * bs:
                    seq.blocks.append(self._take())
                else:
                    last = seq.blocks[pos // bs]
                    if self._ref[last] > 1:  # a partially filled block still shared with the group
                        fresh = self._take()
                        cow.append((last, fresh))
                        self._release(last)
                        seq.blocks[pos // bs] = fresh
                slots[i * num_tokens + t] = seq.blocks[pos // bs] * bs + pos % bs
                seq.length += 1
        return slots, cow

    def blocks_needed(self, seq_ids, num_tokens: int = 1) -> int:
        """Blocks ``append_slots(seq_ids, num_tokens)`` would take from the free pool."""
        return self._append_plan(list(seq_ids), int(num_tokens))

    def any_shared(self, seq_ids) -> bool:
        """Whether any block of these sequences is held by more than one sequence: a
        decode step over them then reads such blocks more than once, and should keep
        them cached (the decode's read policy, ``shared_blocks``)."""
        for sid in seq_ids:
            blocks = self._seqs[sid].blocks
            if blocks and int(self._ref[np.asarray(blocks, dtype=np.int64)].max()) > 1:
                return True
        return False

    def free(self, seq_id) -> None:
        """Release a finished sequence's blocks (indexed prompt blocks stay matchable)."""
        seq = self._seqs.pop(seq_id)
        for b in reversed(seq.blocks):
            self._release(b)

    def sleep(self) -> None:
        """Before the pool's memory is released (the engine's sleep, engine.py:858-869):
        forget every cached prompt block; refuses while sequences still hold blocks."""
        if self._seqs:
            raise RuntimeError(f"{len(self._seqs)} sequences still hold KV blocks: finish or free them before sleep")
        self.reset_prefix_cache()

    def reset_prefix_cache(self) -> None:
        """Forget every cached prompt block (engine.py:864, :1236-1242); live tables are untouched."""
        for b in self._evictable:
            self._free.append(b)
        self._evictable.clear()
        self._index.clear()
        self._hash_of.clear()

    # -- tables ------------------------------------------------------------------
    def __contains__(self, seq_id) -> bool:
        return seq_id in self._seqs

    def seq_len(self, seq_id) -> int:
        return self._seqs[seq_id].length

    def blocks_of(self, seq_id) -> list[int]:
        return list(self._seqs[seq_id].blocks)

    def ref_count(self, block: int) -> int:
        return int(self._ref[block])

    def shared_prefix_tokens(self, seq_ids) -> int:
        """Leading tokens every sequence in ``seq_ids`` reads from the same physical
        blocks: the ``prefix_lens`` entry of a group for ``paged_decode_gqa_grouped``
        (a GRPO group after ``share_prefix`` / ``fork``, engine.py:69-90)."""
        seqs = [self._seqs[s] for s in seq_ids]
        if not seqs:
            return 0
        n = min(len(s.blocks) for s in seqs)
        shared = 0
        while shared < n and all(s.blocks[shared] == seqs[0].blocks[shared] for s in seqs[1:]):
            shared += 1
        return min(shared * self.block_size, min(s.length for s in seqs))

    def tables(self, seq_ids, width: int | None = None) -> tuple[np.ndarray, np.ndarray]:
        """``block_table [B, width]`` int32 (unused entries -1) and ``seq_lens [B]`` int32.

        ``width`` defaults to ``max_blocks_per_seq`` under a ``max_model_len``
        (a fixed shape for every step), else to the longest table."""
        seqs = [self._seqs[s] for s in seq_ids]
        if width is None:
            width = self.max_blocks_per_seq
        w = max((len(s.blocks) for s in seqs), default=1) if width is None else int(width)
        bt = np.full((len(seqs), max(w, 1)), -1, dtype=np.int32)
        for i, s in enumerate(seqs):
            if len(s.blocks) > w:
                raise ValueError(f"width {w} is narrower than a table of {len(s.blocks)} blocks")
            bt[i, :len(s.blocks)] = s.blocks
        lens = np.array([s.length for s in seqs], dtype=np.int32)
        return bt, lens
