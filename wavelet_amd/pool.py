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

import torch

from .blocks import BlockManager
from .cache import MLALatentCache, PagedKVCache


class KVPool:
    """``num_layers`` paged caches of one geometry and the ``BlockManager`` that
    hands out their (shared) block ids."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int = 0, head_dim: int = 0,
                 kv_dtype: str = "bf16", *, mla: bool = False, kv_lora_rank: int = 512, rope_dim: int = 64,
                 enable_prefix_caching: bool = True, device: torch.device | str | None = None) -> None:
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if mla:
            self.layers = [MLALatentCache(num_blocks, block_size, kv_lora_rank, rope_dim, device=device)
                           for _ in range(num_layers)]
        else:
            self.layers = [PagedKVCache(num_blocks, block_size, num_kv_heads, head_dim, kv_dtype, device=device)
                           for _ in range(num_layers)]
        self.blocks = BlockManager(num_blocks, block_size, enable_prefix_caching=enable_prefix_caching)

    @property
    def asleep(self) -> bool:
        return self.layers[0].asleep

    @property
    def nbytes(self) -> int:
        """Device bytes of every layer's pool while awake."""
        return sum(c.nbytes for c in self.layers)

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
