"""The engine-level KV pool: every layer's cache plus the block manager, with
the lifecycle the reference drives.

``VLLMPolicyInferenceEngine`` sizes one pool at setup (engine.py:776-825),
resets its prefix cache after an adapter reload (engine.py:1236-1242), and
between rollout phases releases it -- ``sleep()``: reset the prefix cache, then
``llm.sleep(level=1)``, which discards the KV cache, then
``torch.cuda.empty_cache()`` (engine.py:858-869) -- and restores it with
``wake_up(tags=["kv_cache"])`` after the weights (scheduler.py:3201-3206,
engine.py:871-873). The concurrency controller reads the pool's usage and
capacity from the Prometheus lines of ``metrics_text()``
(wavelet/orchestrator/inference_metrics.py:16-20, :125-133; concurrency.py:43).
"""

from __future__ import annotations

from typing import Callable

import numpy as np
import torch

from .blocks import BlockManager
from .cache import MLALatentCache, PagedKVCache


# Device memory a pool sized from the engine's knobs leaves unclaimed beyond
# ``non_kv_bytes``: the decode split-K workspace, sampler outputs and the
# allocator's rounding.
DEFAULT_RESERVE_BYTES = 512 << 20


def block_bytes(num_layers: int, block_size: int, num_kv_heads: int = 0, head_dim: int = 0, kv_dtype: str = "bf16",
                *, mla: bool = False, kv_lora_rank: int = 512, rope_dim: int = 64) -> int:
    """Device bytes one physical block id holds across every layer (K, V and fp8
    scales, or one MLA latent block)."""
    if mla:
        return num_layers * block_size * (kv_lora_rank + rope_dim) * 2
    elem = 1 if kv_dtype == "fp8_e4m3" else 2
    per_layer = 2 * block_size * num_kv_heads * head_dim * elem
    if kv_dtype == "fp8_e4m3":
        per_layer += 2 * num_kv_heads * 4
    return num_layers * per_layer


class KVPool:
    """``num_layers`` paged caches of one geometry and the ``BlockManager`` that
    hands out their (shared) block ids."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int = 0, head_dim: int = 0,
                 kv_dtype: str = "bf16", *, mla: bool = False, kv_lora_rank: int = 512, rope_dim: int = 64,
                 enable_prefix_caching: bool = True, max_model_len: int | None = None,
                 device: torch.device | str | None = None) -> None:
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if max_model_len is not None and int(max_model_len) > num_blocks * block_size:
            raise ValueError(f"max_model_len {max_model_len} exceeds the pool's {num_blocks * block_size} tokens")
        if mla:
            self.layers = [MLALatentCache(num_blocks, block_size, kv_lora_rank, rope_dim, device=device)
                           for _ in range(num_layers)]
        else:
            # blocks can be shared (prefix caching, or a fork's prompt whether or not prefix caching is
            # on), so a decode without a step-level choice keeps K/V cached between readers; a step
            # whose sequences share nothing streams it instead (decode_shares_blocks)
            self.layers = [PagedKVCache(num_blocks, block_size, num_kv_heads, head_dim, kv_dtype, device=device,
                                        shared_blocks=True)
                           for _ in range(num_layers)]
        self.blocks = BlockManager(num_blocks, block_size, enable_prefix_caching=enable_prefix_caching,
                                   max_model_len=max_model_len)

    @classmethod
    def from_engine_config(cls, *, num_layers: int, num_kv_heads: int = 0, head_dim: int = 0, kv_dtype: str = "bf16",
                           block_size: int = 16, gpu_memory_utilization: float = 0.35,
                           max_model_len: int | None = None, non_kv_bytes: int = 0,
                           reserve_bytes: int = DEFAULT_RESERVE_BYTES, mla: bool = False, kv_lora_rank: int = 512,
                           rope_dim: int = 64, enable_prefix_caching: bool = True,
                           device: torch.device | str | None = None,
                           mem_get_info: Callable[[], tuple[int, int]] | None = None) -> "KVPool":
        """A pool sized the way the engine sizes its KV cache at setup.

        ``gpu_memory_utilization`` (``RLVLLMConfig``, default 0.35, in (0, 1];
        wavelet/configs/config.py:1003-1004, passed to the engine at
        wavelet/inference/engine.py:790-803) is the fraction of the device's
        total memory this engine may hold. Of that share, ``non_kv_bytes``
        (the caller's weights and activations) and ``reserve_bytes`` (the
        path's workspaces and allocator slack) are set aside and the rest
        becomes whole blocks: ``num_gpu_blocks = (utilization * total -
        non_kv_bytes - reserve_bytes) // block_bytes(...)``, the figure
        ``metrics_text()`` then reports. The share must be free when the pool
        is built. ``max_model_len`` (engine.py:809-810; None = no limit below
        the pool's capacity) must fit in the pool, fixes the block-table
        width, and is the longest sequence the block manager admits.
        ``mem_get_info`` returns ``(free, total)`` bytes (default
        ``torch.cuda.mem_get_info``). Raises ValueError when the share is
        not free, holds no block, or cannot hold one ``max_model_len``
        sequence.
        """
        util = float(gpu_memory_utilization)
        if not 0.0 < util <= 1.0:
            raise ValueError(f"gpu_memory_utilization must be in (0, 1] (got {gpu_memory_utilization})")
        if non_kv_bytes < 0 or reserve_bytes < 0:
            raise ValueError("non_kv_bytes and reserve_bytes must be non-negative")
        if max_model_len is not None and int(max_model_len) <= 0:
            raise ValueError(f"max_model_len must be positive (got {max_model_len})")
        if mem_get_info is None:
            dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
            mem_get_info = lambda: torch.cuda.mem_get_info(dev)  # noqa: E731
        free, total = (int(x) for x in mem_get_info())
        requested = int(util * total)
        if requested > free:
            raise ValueError(f"free device memory ({free / 2**30:.2f} GiB) is less than gpu_memory_utilization "
                             f"{util} of {total / 2**30:.2f} GiB ({requested / 2**30:.2f} GiB)")
        per_block = block_bytes(num_layers, block_size, num_kv_heads, head_dim, kv_dtype, mla=mla,
                                kv_lora_rank=kv_lora_rank, rope_dim=rope_dim)
        if per_block <= 0:
            raise ValueError("the cache geometry holds no bytes per block")
        budget = requested - int(non_kv_bytes) - int(reserve_bytes)
        num_blocks = budget // per_block if budget > 0 else 0
        # the decode kernels index (block, KV head) regions with 32-bit integers
        heads = 1 if mla else max(int(num_kv_heads), 1)
        num_blocks = min(num_blocks, (2**31 - 1) // heads)
        if num_blocks <= 0:
            raise ValueError(f"no memory for KV blocks: {requested} bytes requested, {non_kv_bytes} non-KV, "
                             f"{reserve_bytes} reserved, {per_block} bytes per block")
        if max_model_len is not None and num_blocks * block_size < int(max_model_len):
            raise ValueError(f"one sequence of max_model_len {max_model_len} tokens needs "
                             f"{-(-int(max_model_len) // block_size) * per_block / 2**30:.2f} GiB of KV cache, more "
                             f"than the {num_blocks * per_block / 2**30:.2f} GiB available")
        return cls(num_layers, int(num_blocks), block_size, num_kv_heads, head_dim, kv_dtype, mla=mla,
                   kv_lora_rank=kv_lora_rank, rope_dim=rope_dim, enable_prefix_caching=enable_prefix_caching,
                   max_model_len=max_model_len, device=device)

    @property
    def num_blocks(self) -> int:
        return self.blocks.num_blocks

    @property
    def block_size(self) -> int:
        return self.blocks.block_size

    @property
    def max_model_len(self) -> int | None:
        return self.blocks.max_model_len

    @property
    def asleep(self) -> bool:
        return self.layers[0].asleep

    @property
    def nbytes(self) -> int:
        """Device bytes of every layer's pool while awake."""
        return sum(c.nbytes for c in self.layers)

    @property
    def device(self) -> torch.device:
        return self.layers[0].device

    def copy_blocks(self, pairs) -> None:
        """Apply copy-on-write pairs ``(src_block, dst_block)`` (``BlockManager.append_slots``)
        to every layer, GQA or MLA: block ``dst`` becomes a copy of ``src``."""
        m = np.asarray(pairs, dtype=np.int64).reshape(-1, 2)
        if m.shape[0] == 0:
            return
        dm = torch.from_numpy(m).to(self.device)
        for c in self.layers:
            c.copy_blocks(dm)

    def append_slots(self, seq_ids, num_tokens: int = 1) -> torch.Tensor:
        """Reserve the step's token slots (``BlockManager.append_slots``), apply its
        copy-on-write pairs to every layer, and return the slot mapping (int64, on the
        pool's device, sequence-major) for the step's appends."""
        slots, cow = self.blocks.append_slots(seq_ids, num_tokens)
        self.copy_blocks(cow)
        return torch.from_numpy(slots).to(self.device)

    def decode_shares_blocks(self, seq_ids) -> bool:
        """The read policy of a decode step over ``seq_ids``: True when some block is held by
        more than one of the pool's sequences (reads then keep K/V cached for the next
        reader), False when every block is read once (reads stream past the caches)."""
        return self.blocks.any_shared(seq_ids)

    def reset_prefix_cache(self) -> None:
        """Forget cached prompt blocks (after a policy or adapter reload, engine.py:1236-1242)."""
        self.blocks.reset_prefix_cache()

    def sleep(self, level: int = 1) -> None:
        """Discard the KV cache and release its device memory. Levels 1 and 2
        treat the KV pool alike (level 2 also drops weights, which live elsewhere)."""
        if level not in (1, 2):
            raise ValueError(f"sleep level must be 1 or 2 (got {level})")
        if self.asleep:
            return
        self.blocks.sleep()
        for c in self.layers:
            c.sleep()
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    def wake_up(self, tags: list[str] | None = None) -> None:
        """Restore the pool (zeroed). ``tags`` as the engine passes them: None or
        a list containing ``"kv_cache"`` wakes the KV pool; ``["weights"]`` alone
        concerns the model weights and leaves the pool asleep."""
        if tags is not None:
            unknown = set(tags) - {"weights", "kv_cache"}
            if unknown:
                raise ValueError(f"unknown wake_up tags {sorted(unknown)}")
            if "kv_cache" not in tags:
                return
        for c in self.layers:
            c.wake_up()

    def metrics_text(self) -> str:
        """``vllm:kv_cache_usage_perc`` and ``vllm:cache_config_info`` lines."""
        return self.blocks.metrics_text()
