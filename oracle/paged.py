"""Paged KV cache semantics restated in numpy (oracle; tests and CPU baseline only).

Slot convention (vLLM's, reached from wavelet/inference/engine.py:887): slot
``s = block_id * block_size + offset``; ``s = -1`` marks a padded token that is
never written. Caches are held in the same physical layout as the HIP library:

* bf16 / fp8 K: ``[num_blocks, H, D // x, block_size, x]``, ``x = 16 // elem_size``
* bf16 / fp8 V: ``[num_blocks, H, D, block_size]``
* fp8 scales:   ``[num_blocks, H]`` fp32 for K and for V
* MLA latent:   ``[num_blocks, block_size, 576]``

bf16 values are carried as uint16 bit patterns and fp8 values as uint8 codes,
so "bit-exact" comparisons are plain integer equality. The layout helpers give
the logical ``[num_blocks, block_size, H, D]`` view every function works on.
"""

from __future__ import annotations

import math

import numpy as np

from . import fp8


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """RNE fp32 -> bf16 bits (NaN stays NaN), torch's ``.to(torch.bfloat16)``."""
    f = np.asarray(x, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    r = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    r = np.where(np.isnan(f), (b >> np.uint64(16)) | np.uint64(0x40), r)
    return r.astype(np.uint16)


# ---------------------------------------------------------------------------
# Layout

def x_of(elem_bytes: int) -> int:
    return 16 // elem_bytes


def k_logical(k_phys: np.ndarray) -> np.ndarray:
    """[NB, H, D/x, BS, x] -> view [NB, BS, H, D/x, x]."""
    return k_phys.transpose(0, 3, 1, 2, 4)


def v_logical(v_phys: np.ndarray) -> np.ndarray:
    """[NB, H, D, BS] -> view [NB, BS, H, D]."""
    return v_phys.transpose(0, 3, 1, 2)


def empty_cache(num_blocks: int, block_size: int, heads: int, head_dim: int, dtype=np.uint16, fill=0):
    x = x_of(np.dtype(dtype).itemsize)
    k = np.full((num_blocks, heads, head_dim // x, block_size, x), fill, dtype=dtype)
    v = np.full((num_blocks, heads, head_dim, block_size), fill, dtype=dtype)
    return k, v


def logical_kv(k_phys: np.ndarray, v_phys: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Contiguous logical copies [NB, BS, H, D] of both caches."""
    nb, h, dx, bs, x = k_phys.shape
    k = np.ascontiguousarray(k_logical(k_phys)).reshape(nb, bs, h, dx * x)
    v = np.ascontiguousarray(v_logical(v_phys))
    return k, v


# ---------------------------------------------------------------------------
# Append

def append_bf16(k_phys, v_phys, key_bits, value_bits, slot_mapping) -> None:
    """``cache.view(NB*BS, H, D)[slot[t]] = x[t]`` for every ``slot[t] >= 0`` (in place).

    Semantics of the cache update the engine performs before attention
    (``past_key_values.update`` at wavelet/kernels/patch.py:173-180; vLLM's
    slot-mapped append inside ``llm.generate``, engine.py:887).
    """
    nb, h, dx, bs, x = k_phys.shape
    slots = np.asarray(slot_mapping, dtype=np.int64)
    keep = slots >= 0
    s = slots[keep]
    blk, off = s // bs, s % bs
    kl, vl = k_logical(k_phys), v_logical(v_phys)
    kl[blk, off] = np.asarray(key_bits)[keep].reshape(-1, h, dx, x)
    vl[blk, off] = np.asarray(value_bits)[keep]


def _runs(slots: np.ndarray, block_size: int):
    """Maximal runs of consecutive valid tokens that land in the same block."""
    t, n = 0, len(slots)
    while t < n:
        if slots[t] < 0:
            t += 1
            continue
        blk = slots[t] // block_size
        r = 1
        while t + r < n and slots[t + r] >= 0 and slots[t + r] // block_size == blk:
            r += 1
        yield t, r, int(blk)
        t += r


def _abs_amax(x: np.ndarray) -> np.float32:
    """max |x| with NaN ignored (IEEE maxNum), as the kernel's fmaxf reduction."""
    a = np.abs(np.asarray(x, dtype=np.float32))
    a = a[~np.isnan(a)]
    return np.float32(a.max()) if a.size else np.float32(0.0)


def append_fp8(k_phys, v_phys, k_scale, v_scale, key_bits, value_bits, slot_mapping) -> None:
    """fp8-e4m3 append with one power-of-two fp32 scale per (block, head), in place.

    Quantisation is the reference's ``_fp8_roundtrip`` convention
    (wavelet/trainer/models/deepseek_v4/attention.py:41-50) applied to a
    (block, head) group instead of a last-dim row. Tokens are handled in runs:
    a run is a maximal stretch of consecutive tokens of this call whose slots
    fall in the same block (a block manager fills a block in slot order, so a
    decode append is a run of one and a prefill writes whole-block runs). For
    each run and head, separately for K and V:

    1. ``s_new = pow2_scale(max |x|)`` over the run's tokens (NaN ignored).
    2. If the run starts at offset 0 the block is fresh: ``s = s_new``.
       Otherwise ``s = max(s_old, s_new)``; when ``s > s_old`` the entries at
       offsets ``[0, first_offset)`` are re-encoded as
       ``e4m3(decode(code) * (s_old / s))`` -- an exact power-of-two shift that
       only rounds (RNE) where the result drops into the e4m3 subnormals.
    3. The run's tokens are stored as ``e4m3(clamp(x / s, +-448))`` and ``s``
       is written back.

    A block must appear in at most one run per call (distinct slots).
    """
    nb, h, dx, bs, x = k_phys.shape
    d = dx * x
    slots = np.asarray(slot_mapping, dtype=np.int64)
    key = bf16_to_f32(key_bits)
    val = bf16_to_f32(value_bits)
    kl, vl = k_logical(k_phys), v_logical(v_phys)
    for t, r, blk in _runs(slots, bs):
        offs = slots[t : t + r] % bs
        first = int(offs[0])
        for src, lview, scales in ((key, kl, k_scale), (val, vl, v_scale)):
            for hh in range(h):
                rows = src[t : t + r, hh, :]  # [r, D]
                s_new = fp8.pow2_scale(_abs_amax(rows))
                if first == 0:
                    s = s_new
                else:
                    s_old = np.float32(scales[blk, hh])
                    s = np.float32(max(s_old, s_new))
                    if s > s_old and first > 0:
                        old = lview[blk, :first, hh].reshape(first, d)
                        ratio = np.float32(s_old / s)
                        new = fp8.e4m3_encode((fp8.e4m3_decode(old) * ratio).astype(np.float32))
                        lview[blk, :first, hh] = new.reshape(lview[blk, :first, hh].shape)
                codes = fp8.quantize(rows, s)
                lview[blk, offs, hh] = codes.reshape((r,) + lview.shape[3:])
                scales[blk, hh] = s


# ---------------------------------------------------------------------------
# Gather

def gather(k_phys, v_phys, block_table, seq_lens):
    """Contiguous ``[sum L, H, D]`` copies: ``out[i, t] = cache[bt[i, t // BS], t % BS]``.

    Block-table read as in ``SparseAttnInputs`` (attention.py:320-360) with the
    gather of attention.py:85-88: entries past ``seq_lens[i]`` are never read.
    Returns raw stored elements (bf16 bits or fp8 codes).
    """
    kl, vl = logical_kv(k_phys, v_phys)
    bs = kl.shape[1]
    outs_k, outs_v = [], []
    for i, length in enumerate(np.asarray(seq_lens, dtype=np.int64)):
        pos = np.arange(length)
        blk = np.asarray(block_table[i], dtype=np.int64)[pos // bs]
        outs_k.append(kl[blk, pos % bs])
        outs_v.append(vl[blk, pos % bs])
    h, d = kl.shape[2], kl.shape[3]
    if not outs_k:
        return np.zeros((0, h, d), kl.dtype), np.zeros((0, h, d), vl.dtype)
    return np.concatenate(outs_k), np.concatenate(outs_v)


def copy_blocks(arrays, pairs) -> None:
    """Copy-on-write block copies, in place: for each ``(src, dst)``, block
    ``dst`` of every array (K, V, scales, or an MLA latent cache; block index
    on axis 0) becomes a copy of block ``src``; pairs naming a block outside
    ``[0, num_blocks)`` are skipped. Pairs are independent -- no block is the
    destination of one pair and the source or destination of another, as the
    block manager's pairs (a shared block, a fresh one) never are -- so every
    copy reads the blocks as they were before the call. vLLM's
    ``copy_blocks``, applied before a GRPO member writes into a prompt block it
    still shares (``SamplingParams(n=...)``, wavelet/inference/engine.py:69-90)."""
    m = np.asarray(pairs, dtype=np.int64).reshape(-1, 2)
    dsts = [int(d) for _, d in m]
    if len(set(dsts)) != len(dsts) or set(dsts) & {int(s) for s, _ in m}:
        raise ValueError("copy pairs must be independent (a destination is never another pair's block)")
    for a in arrays:
        before = a.copy()
        for src, dst in m:
            if 0 <= src < a.shape[0] and 0 <= dst < a.shape[0]:
                a[dst] = before[src]


def append_mla(latent, kv_c_bits, k_pe_bits, slot_mapping) -> None:
    """``latent.view(NB*BS, R+P)[slot[t]] = concat(kv_c[t], k_pe[t])`` for every
    ``slot[t] >= 0`` (in place): vLLM's ``concat_and_cache_mla`` on the
    ``[NB, BS, R + P]`` latent layout (the row the DSV4 shared-KV attention
    keeps per token, wavelet/trainer/models/deepseek_v4/attention.py:652-663)."""
    nb, bs, w = latent.shape
    r = kv_c_bits.shape[1]
    flat = latent.reshape(nb * bs, w)
    for t, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64)):
        if 0 <= slot < nb * bs:
            flat[slot, :r] = kv_c_bits[t]
            flat[slot, r:] = k_pe_bits[t]


def gather_mla(latent, block_table, seq_lens) -> np.ndarray:
    """Contiguous ``[sum L, R + P]`` copy of each sequence's latent rows:
    ``out[i, t] = latent[bt[i, t // BS], t % BS]`` for ``t < seq_lens[i]`` (the
    index read of ``SparseAttnInputs``, attention.py:320-360, and the gather of
    attention.py:85-88 over the shared latent); entries past ``seq_lens[i]`` are
    never read. Raw stored elements (bf16 bits)."""
    bs, w = latent.shape[1], latent.shape[2]
    parts = []
    for i, length in enumerate(np.asarray(seq_lens, dtype=np.int64)):
        pos = np.arange(length)
        parts.append(latent[np.asarray(block_table[i], dtype=np.int64)[pos // bs], pos % bs])
    return np.concatenate(parts) if parts else np.zeros((0, w), latent.dtype)


def dequant_gathered(codes: np.ndarray, scales: np.ndarray, block_table, seq_lens, block_size) -> np.ndarray:
    """fp8 codes from ``gather`` -> fp32 values, scale of each token's (block, head)."""
    parts = []
    for i, length in enumerate(np.asarray(seq_lens, dtype=np.int64)):
        pos = np.arange(length)
        blk = np.asarray(block_table[i], dtype=np.int64)[pos // block_size]
        parts.append(scales[blk][:, :, None])
    s = np.concatenate(parts) if parts else np.zeros((0, codes.shape[1], 1), np.float32)
    return fp8.dequantize(codes, s)


# ---------------------------------------------------------------------------
# Attention

def _softmax_rows(s: np.ndarray, sink=None) -> np.ndarray:
    """Row softmax; with ``sink`` (one logit per row) each row's softmax also
    holds that logit, whose probability is dropped: the learned zero-value sink
    of wavelet/trainer/models/deepseek_v4/attention.py:89-95 (scores
    concatenated with the sink, softmax, last column removed)."""
    m = s.max(axis=-1, keepdims=True)
    if sink is None:
        e = np.exp(s - m)
        return e / e.sum(axis=-1, keepdims=True)
    sink = np.asarray(sink, dtype=s.dtype).reshape(-1, 1)
    m = np.maximum(m, sink)
    e = np.exp(s - m)
    return e / (e.sum(axis=-1, keepdims=True) + np.exp(sink - m))


def decode_gqa(q, k_vals, v_vals, block_table, seq_lens, scale, *, p_bf16=False, dtype=np.float64, sinks=None):
    """GQA paged decode: ``o[i, h] = softmax(q[i,h] . K_i^T * scale) . V_i``.

    ``q`` is ``[B, Hq, D]`` values; ``k_vals``/``v_vals`` are logical
    ``[NB, BS, Hkv, D]`` *values* (bf16 widened, or fp8 already dequantised).
    Query head ``h`` reads KV head ``h // (Hq // Hkv)``. Scores and softmax in
    ``dtype`` (fp32 scores/softmax as at attention.py:89-93); with ``p_bf16``
    the probabilities are rounded to bf16 before PV, as attention.py:94-96 casts
    them to the KV dtype (the reference bf16 path). ``sinks`` (``[Hq]``,
    natural-log logits, ``-inf`` = none) adds each head's zero-value sink
    logit to its softmax (``_softmax_rows``). A zero-length sequence gives
    zeros. Returns ``[B, Hq, D]`` in ``dtype``.
    """
    q = np.asarray(q)
    b, hq, d = q.shape
    nb, bs, hkv, _ = k_vals.shape
    g = hq // hkv
    out = np.zeros((b, hq, d), dtype=dtype)
    for i in range(b):
        length = int(seq_lens[i])
        if length == 0:
            continue
        pos = np.arange(length)
        blk = np.asarray(block_table[i], dtype=np.int64)[pos // bs]
        kk = k_vals[blk, pos % bs].astype(dtype)  # [L, Hkv, D]
        vv = v_vals[blk, pos % bs].astype(dtype)
        for h in range(hkv):
            qh = q[i, h * g : (h + 1) * g].astype(dtype)  # [G, D]
            sink = None if sinks is None else np.asarray(sinks, dtype=dtype)[h * g : (h + 1) * g]
            p = _softmax_rows((qh @ kk[:, h].T) * dtype(scale), sink)
            if p_bf16:
                p = bf16_to_f32(f32_to_bf16(p.astype(np.float32))).astype(dtype)
            out[i, h * g : (h + 1) * g] = p @ vv[:, h]
    return out


def prefill_gqa(q, k_vals, v_vals, block_table, seq_lens, cu_seqlens_q, scale, *, p_bf16=False, dtype=np.float64,
                sinks=None):
    """Varlen GQA prefill over a paged context (chunked prefill).

    Sequence ``i`` brings ``n_i = cu_seqlens_q[i+1] - cu_seqlens_q[i]`` new
    tokens, rows ``cu_seqlens_q[i] ..`` of ``q`` ``[T, Hq, D]``, at positions
    ``L_i - n_i .. L_i - 1`` (``L_i = seq_lens[i]`` counts the cached context
    and the new tokens, whose K/V are already in the cache). New token ``j``
    attends to positions ``0 .. L_i - n_i + j``: the causal mask of the
    engine's prompt step (``llm.generate``, wavelet/inference/engine.py:887)
    aligned to the end of the context, so an earlier chunk or a prefix-cache
    hit is simply cached context. Scores, softmax and ``sinks`` as in
    ``decode_gqa``.
    Returns ``[T, Hq, D]`` in ``dtype``.
    """
    q = np.asarray(q)
    t, hq, d = q.shape
    nb, bs, hkv, _ = k_vals.shape
    g = hq // hkv
    out = np.zeros((t, hq, d), dtype=dtype)
    for i in range(len(seq_lens)):
        q0, q1 = int(cu_seqlens_q[i]), int(cu_seqlens_q[i + 1])
        n, length = q1 - q0, int(seq_lens[i])
        if n == 0 or length == 0:
            continue
        pos = np.arange(length)
        blk = np.asarray(block_table[i], dtype=np.int64)[pos // bs]
        kk = k_vals[blk, pos % bs].astype(dtype)  # [L, Hkv, D]
        vv = v_vals[blk, pos % bs].astype(dtype)
        qpos = length - n + np.arange(n)  # [n]
        mask = pos[None, :] <= qpos[:, None]  # [n, L]
        for h in range(hkv):
            for hh in range(h * g, (h + 1) * g):
                s = (q[q0:q1, hh].astype(dtype) @ kk[:, h].T) * dtype(scale)  # [n, L]
                s = np.where(mask, s, -np.inf)
                p = _softmax_rows(s, None if sinks is None else np.full(n, sinks[hh], dtype=dtype))
                if p_bf16:
                    p = bf16_to_f32(f32_to_bf16(p.astype(np.float32))).astype(dtype)
                out[q0:q1, hh] = p @ vv[:, h]
    return out


def decode_mla(q, latent_vals, block_table, seq_lens, scale, kv_lora_rank=512, *, p_bf16=False, dtype=np.float64,
               sinks=None):
    """Weight-absorbed MLA decode over a single latent head.

    ``q`` ``[B, H, R + P]`` (absorbed ``q_nope @ W_UK`` then ``q_pe``),
    ``latent_vals`` logical ``[NB, BS, R + P]`` (``c_kv`` then ``k_pe``):
    ``s = q . c^T * scale``; ``o_lat = softmax(s) . c[:, :R]``. Every query
    head shares the one latent entry, as the DSV4 shared-KV MQA does
    (attention.py:652-663, 744-771). ``sinks`` (``[H]``, natural-log logits,
    ``-inf`` = none) adds each head's zero-value sink logit to its softmax, as
    that attention's per-head ``sinks`` (attention.py:703, used at :89-95 and
    :763) do. A zero-length sequence gives zeros. Returns ``[B, H, R]``.
    """
    q = np.asarray(q)
    b, h, w = q.shape
    nb, bs, _ = latent_vals.shape
    out = np.zeros((b, h, kv_lora_rank), dtype=dtype)
    for i in range(b):
        length = int(seq_lens[i])
        if length == 0:
            continue
        pos = np.arange(length)
        blk = np.asarray(block_table[i], dtype=np.int64)[pos // bs]
        c = latent_vals[blk, pos % bs].astype(dtype)  # [L, R+P]
        p = _softmax_rows((q[i].astype(dtype) @ c.T) * dtype(scale),
                          None if sinks is None else np.asarray(sinks, dtype=dtype))
        if p_bf16:
            p = bf16_to_f32(f32_to_bf16(p.astype(np.float32))).astype(dtype)
        out[i] = p @ c[:, :kv_lora_rank]
    return out


def max_abs_and_rel(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    """(max |got - ref|, ||got - ref||_2 / ||ref||_2) in float64."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    diff = g - r
    denom = math.sqrt(float((r * r).sum())) or 1.0
    return float(np.abs(diff).max()) if diff.size else 0.0, math.sqrt(float((diff * diff).sum())) / denom
