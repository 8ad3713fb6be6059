"""The reference's own attention call convention on the paged path.

The Qwen3 attention forward that the reference patches (wavelet/kernels/patch.py:173-196,
the same sequence as transformers' own) runs, per layer and step::

    key_states, value_states = past_key_values.update(key_states, value_states, self.layer_idx, cache_kwargs)
    attention_interface = ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation, ...)
    attn_output, attn_weights = attention_interface(self, query_states, key_states, value_states,
                                                    attention_mask, dropout=..., scaling=self.scaling, ...)

Here ``past_key_values`` is a ``PagedCache`` (a transformers ``Cache`` whose batch rows are
sequences of a ``KVPool``) and the attention implementation is ``"wavelet_paged"``
(``register()``): a layer's ``update`` keeps the step's key/value rows and returns them tagged
with the cache; the attention call then appends them to the layer's paged cache and attends in
one launch -- ``prefill_gqa`` for a step of several tokens per row (the prompt, or a chunk after
cached context), the fused append + ``paged_decode_gqa`` for one token per row. The causal mask
comes from the sequences' lengths (bottom-right aligned), so no dense mask is built.

Scope: every row brings the same number of tokens per step and holds no padding (a model run
on equal-length rows, as GRPO's n samples of one prompt are); beam search, sliding windows,
dropout and attention weights are not supported and raise.
"""

from __future__ import annotations

import itertools

import numpy as np
import torch
from transformers import AttentionInterface
from transformers.cache_utils import Cache, CacheLayerMixin
from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

from .attention import paged_decode_gqa, prefill_gqa
from .cache import PagedKVCache
from .pool import KVPool

ATTN_IMPLEMENTATION = "wavelet_paged"
_salts = itertools.count()


class _PagedLayer(CacheLayerMixin):
    """One layer of a PagedCache: its tokens live in the pool's cache of that layer."""

    is_compileable = False

    def __init__(self, owner: "PagedCache", layer_idx: int) -> None:
        super().__init__()
        self._owner = owner
        self._layer = layer_idx
        self.seen = 0  # tokens of each row this layer holds

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        return self._owner._stage(self._layer, key_states, value_states)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.seen + query_length, 0

    def get_seq_length(self) -> int:
        return self.seen

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        raise NotImplementedError("a PagedCache is not reset in place: free its sequences and build a new one")

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        raise NotImplementedError("beam search reorders rows, which the paged cache does not support")


class PagedCache(Cache):
    """transformers ``Cache`` over a ``KVPool``: batch row ``i`` is sequence ``seq_ids[i]`` of the
    pool's block manager (allocated at its first step when new; an existing sequence -- a
    cached prompt, an earlier chunk, a GRPO fork -- continues where it stands).

    Each model step reserves the step's token slots once (its first layer's ``update``), applies
    the block manager's copy-on-write pairs to every layer, and hands every layer the same
    block table, lengths and slot mapping; the step's decodes keep K/V cached only when some
    block is held by more than one row (``BlockManager.any_shared``), else they stream it.
    Use with ``attn_implementation="wavelet_paged"``.
    """

    def __init__(self, pool: KVPool, seq_ids) -> None:
        if not pool.layers or not isinstance(pool.layers[0], PagedKVCache):
            raise ValueError("PagedCache needs a GQA KVPool (PagedKVCache layers)")
        super().__init__(layers=[_PagedLayer(self, i) for i in range(len(pool.layers))])
        self.pool = pool
        self.seq_ids = list(seq_ids)
        if not self.seq_ids or len(set(self.seq_ids)) != len(self.seq_ids):
            raise ValueError("seq_ids must be distinct and non-empty")
        self._step: dict | None = None
        self._staged: set[int] = set()
        self._pending: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        self._salt = f"hf-paged-{next(_salts)}"

    # -- the step's slots -------------------------------------------------------------
    def _begin_step(self, tokens: int, device: torch.device) -> None:
        if self._pending:
            raise RuntimeError(f"layers {sorted(self._pending)} were updated but never attended: the attention "
                               f"implementation must be {ATTN_IMPLEMENTATION!r}")
        bm, bs = self.pool.blocks, self.pool.block_size
        old_rows = [sid for sid in self.seq_ids if sid in bm]
        new_rows = [sid for sid in self.seq_ids if sid not in bm]
        # every check before any state moves: a step that cannot be taken leaves the manager as it was
        if new_rows and bm.max_model_len is not None and tokens > bm.max_model_len:
            raise ValueError(f"a new sequence of {tokens} tokens is longer than max_model_len {bm.max_model_len}")
        need = bm.blocks_needed(old_rows, tokens) + len(new_rows) * -(-tokens // bs)
        if need > bm.num_free_blocks:
            raise MemoryError(f"out of KV cache blocks: the step needs {need}, {bm.num_free_blocks} are free")
        rows: dict = {}
        if old_rows:
            s, cow = bm.append_slots(old_rows, tokens)
            for i, sid in enumerate(old_rows):
                rows[sid] = s[i * tokens:(i + 1) * tokens]
            # a row about to write into a block it still shares gets its own copy first
            self.pool.copy_blocks(cow)
        pos = np.arange(tokens)
        for sid in new_rows:
            # a new sequence: its prompt's blocks (token ids unseen here, so a private salt
            # keeps the prefix index from matching them)
            bm.allocate(sid, np.zeros(tokens, dtype=np.int64), cache_salt=f"{self._salt}-{sid}")
            rows[sid] = np.asarray(bm.blocks_of(sid), dtype=np.int64)[pos // bs] * bs + pos % bs
        slots = np.stack([rows[sid] for sid in self.seq_ids])
        bt, sl = bm.tables(self.seq_ids)
        self._step = {
            "tokens": tokens,
            "slots": torch.from_numpy(slots.reshape(-1)).to(device),
            "block_table": torch.from_numpy(bt).to(device),
            "seq_lens": torch.from_numpy(sl).to(device),
            "cu_seqlens_q": torch.arange(0, len(self.seq_ids) * tokens + 1, tokens, dtype=torch.int32, device=device),
            "max_seq_len": int(sl.max()),
            # blocks held by more than one row are read more than once: keep them cached
            "shared_blocks": bm.any_shared(self.seq_ids),
        }
        self._staged.clear()

    def _stage(self, layer: int, key_states: torch.Tensor, value_states: torch.Tensor):
        if key_states.dim() != 4 or key_states.shape != value_states.shape:
            raise ValueError("key/value states must be [batch, kv_heads, tokens, head_dim] and alike")
        b, _, tokens, _ = key_states.shape
        if b != len(self.seq_ids):
            raise ValueError(f"batch of {b} rows for a cache of {len(self.seq_ids)} sequences")
        if layer == 0 or self._step is None or layer in self._staged:
            self._begin_step(tokens, key_states.device)
        elif tokens != self._step["tokens"]:
            raise ValueError("every layer of a step brings the same tokens")
        self._staged.add(layer)
        self._pending[layer] = (key_states, value_states)
        k, v = key_states.view_as(key_states), value_states.view_as(value_states)
        k._wavelet_paged = v._wavelet_paged = (self, layer)
        return k, v

    def _attend(self, layer: int, query: torch.Tensor, scale: float,
                sinks: torch.Tensor | None = None) -> torch.Tensor:
        k, v = self._pending.pop(layer)
        st = self._step
        b, hq, tokens, d = query.shape
        hkv = k.shape[1]
        q = query.transpose(1, 2).reshape(b * tokens, hq, d).contiguous()
        kk = k.transpose(1, 2).reshape(b * tokens, hkv, d).contiguous()
        vv = v.transpose(1, 2).reshape(b * tokens, hkv, d).contiguous()
        cache = self.pool.layers[layer]
        if tokens == 1:
            out = paged_decode_gqa(q, cache, st["block_table"], st["seq_lens"], scale, max_seq_len=st["max_seq_len"],
                                   new_key=kk, new_value=vv, slot_mapping=st["slots"], sinks=sinks,
                                   shared_blocks=st["shared_blocks"])
        else:
            out = prefill_gqa(q, cache, st["block_table"], st["seq_lens"], st["cu_seqlens_q"], scale, key=kk,
                              value=vv, slot_mapping=st["slots"], max_query_len=tokens,
                              max_seq_len=st["max_seq_len"], sinks=sinks)
        self.layers[layer].seen += tokens
        return out.view(b, tokens, hq, d)


def paged_attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            attention_mask: torch.Tensor | None, scaling: float | None = None, dropout: float = 0.0,
                            sliding_window: int | None = None, **kwargs):
    """``attention_interface`` for ``"wavelet_paged"``: ``query [B, Hq, T, D]`` and the key/value
    that ``PagedCache.update`` returned -> ``([B, T, Hq, D], None)``. ``s_aux`` (a model's per-head
    attention sinks, as transformers passes them) becomes the kernels' ``sinks``."""
    tag = getattr(key, "_wavelet_paged", None)
    if tag is None:
        raise ValueError(f"{ATTN_IMPLEMENTATION!r} attention needs the key/value states PagedCache.update returned")
    if dropout:
        raise NotImplementedError("dropout is not supported on the paged path")
    if sliding_window is not None:
        raise NotImplementedError("sliding-window attention is not supported on the paged path")
    cache, layer = tag
    scale = float(scaling) if scaling is not None else query.shape[-1] ** -0.5
    s_aux = kwargs.get("s_aux")
    sinks = None if s_aux is None else s_aux.detach().to(device=query.device, dtype=torch.float32).contiguous()
    return cache._attend(layer, query, scale, sinks), None


def _no_mask(*args, **kwargs):
    """The paged kernels mask causally from the sequences' lengths: no dense mask is built."""
    return None


def register() -> str:
    """Register ``"wavelet_paged"`` with transformers' attention and mask interfaces; returns the name."""
    AttentionInterface.register(ATTN_IMPLEMENTATION, paged_attention_forward)
    ALL_MASK_ATTENTION_FUNCTIONS.register(ATTN_IMPLEMENTATION, _no_mask)
    return ATTN_IMPLEMENTATION
