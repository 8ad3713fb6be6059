"""Seeded synthetic workloads for the paged KV-cache decode path.

Every random tensor comes from a repo-local counter-based generator
(splitmix64 -> Box-Muller), keyed by ``(workload, tensor name)``. The bytes
therefore do not depend on the torch or numpy RNG implementations, and the CPU
test container and the GPU host produce identical inputs; ``sha256_of``
fingerprints them so a test can prove it.

The workloads follow the engine's decode loop (``llm.generate`` at
wavelet/inference/engine.py:887, :1045, :1274): each running sequence owns a
block table of physical cache blocks; a decode step appends one token per
sequence into slot ``block_id * block_size + offset`` and then attends over the
sequence's whole context through its block table.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser on a uint64 array (wrapping arithmetic)."""
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(*names: object) -> int:
    """64-bit key for a named random stream (FNV-1a over the joined names)."""
    h = 0xCBF29CE484222325
    for byte in "/".join(str(n) for n in names).encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def random_u64(key: int, n: int, offset: int = 0) -> np.ndarray:
    """Counter-based uint64 stream: element i is splitmix64(key + (offset+i+1)*golden)."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        return _mix(np.uint64(key) + idx * _GOLDEN)


def uniform01(key: int, n: int, offset: int = 0) -> np.ndarray:
    """Uniform doubles in (0, 1] with 53 random bits."""
    bits = random_u64(key, n, offset) >> np.uint64(11)
    return (bits.astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(key: int, n: int) -> np.ndarray:
    """Standard normal doubles by Box-Muller over consecutive uniform pairs."""
    m = (n + 1) // 2
    u = uniform01(key, 2 * m)
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    t = 2.0 * np.pi * u[1::2]
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n]


def randint(key: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi] (inclusive), via the high 32 bits times range."""
    span = np.uint64(hi - lo + 1)
    hi32 = random_u64(key, n) >> np.uint64(32)
    return (lo + ((hi32 * span) >> np.uint64(32)).astype(np.int64)).astype(np.int64)


def permutation(key: int, n: int) -> np.ndarray:
    """Seeded permutation of 0..n-1 (stable argsort of random 64-bit keys)."""
    return np.argsort(random_u64(key, n), kind="stable").astype(np.int64)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float64/float32 values to bf16 (RNE, NaN kept) and return uint16 bits."""
    f = np.asarray(x, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    rounded = np.where(nan, (b >> np.uint64(16)) | np.uint64(0x40), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(key: int, shape: tuple[int, ...], std: float = 1.0) -> np.ndarray:
    """bf16 bit patterns (uint16) of N(0, std^2) samples of the given shape."""
    n = int(np.prod(shape)) if shape else 1
    return to_bf16_bits(normal(key, n) * std).reshape(shape)


def sha256_of(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@dataclass
class DecodeWorkload:
    """One layer's worth of decode-step inputs in the engine's own terms.

    ``context_lens`` are the lengths *after* this step's append, so the new
    token of sequence i lands at position ``context_lens[i] - 1``. Caches hold
    ``context_lens[i] - 1`` previously written tokens per sequence.
    """

    name: str
    num_blocks: int
    block_size: int
    num_kv_heads: int
    num_q_heads: int
    head_dim: int
    context_lens: np.ndarray  # [B] int32
    block_tables: np.ndarray  # [B, max_blocks] int32, unused entries -1
    scale: float
    group_size: int = 1  # sequences per prompt group sharing the prefix blocks
    prefix_len: int = 0  # tokens shared by each group (whole blocks)
    extras: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.context_lens.shape[0])

    @property
    def max_blocks(self) -> int:
        return int(self.block_tables.shape[1])

    def new_token_slots(self) -> np.ndarray:
        pos = self.context_lens.astype(np.int64) - 1
        blk = self.block_tables[np.arange(self.batch), pos // self.block_size].astype(np.int64)
        return blk * self.block_size + pos % self.block_size


def _deal_blocks(perm: np.ndarray, nblocks_per_seq: np.ndarray, width: int) -> np.ndarray:
    """Deal a permutation of physical blocks to sequences in order."""
    bt = np.full((len(nblocks_per_seq), width), -1, dtype=np.int32)
    cursor = 0
    for i, nb in enumerate(nblocks_per_seq):
        bt[i, :nb] = perm[cursor : cursor + nb]
        cursor += nb
    return bt


def make_decode_workload(
    name: str,
    *,
    batch: int,
    num_kv_heads: int,
    num_q_heads: int,
    head_dim: int,
    block_size: int,
    context_lens: np.ndarray,
    num_blocks: int | None = None,
    scale: float | None = None,
) -> DecodeWorkload:
    """Independent sequences, block tables dealt from a seeded permutation."""
    context_lens = np.asarray(context_lens, dtype=np.int32)
    assert context_lens.shape == (batch,)
    nb_seq = (context_lens.astype(np.int64) + block_size - 1) // block_size
    need = int(nb_seq.sum())
    num_blocks = need if num_blocks is None else num_blocks
    if num_blocks < need:
        raise ValueError(f"{name}: {need} blocks needed, pool has {num_blocks}")
    perm = permutation(stream_key(name, "block_perm"), num_blocks)
    width = int(nb_seq.max()) if batch else 1
    bt = _deal_blocks(perm, nb_seq, width)
    return DecodeWorkload(
        name=name,
        num_blocks=num_blocks,
        block_size=block_size,
        num_kv_heads=num_kv_heads,
        num_q_heads=num_q_heads,
        head_dim=head_dim,
        context_lens=context_lens,
        block_tables=bt,
        scale=(1.0 / np.sqrt(head_dim)) if scale is None else scale,
    )


def make_group_workload(
    name: str,
    *,
    num_groups: int,
    group_size: int,
    prefix_len: int,
    gen_lens: np.ndarray,
    num_kv_heads: int,
    num_q_heads: int,
    head_dim: int,
    block_size: int,
    num_blocks: int | None = None,
) -> DecodeWorkload:
    """GRPO-style groups: ``group_size`` sequences share a ``prefix_len``-token prompt.

    The prompt's whole blocks are one set of physical blocks referenced by every
    member's block table (the n>1 sampling of ``vllm_sampling_kwargs``,
    wavelet/inference/engine.py:69-90); each member's generated tokens live in
    private blocks. ``gen_lens[i]`` counts generated tokens including this step's.
    """
    if prefix_len % block_size:
        raise ValueError("shared prefix must be whole blocks")
    batch = num_groups * group_size
    gen_lens = np.asarray(gen_lens, dtype=np.int64)
    assert gen_lens.shape == (batch,)
    pb = prefix_len // block_size
    priv = (gen_lens + block_size - 1) // block_size
    need = num_groups * pb + int(priv.sum())
    num_blocks = need if num_blocks is None else num_blocks
    if num_blocks < need:
        raise ValueError(f"{name}: {need} blocks needed, pool has {num_blocks}")
    perm = permutation(stream_key(name, "block_perm"), num_blocks)
    width = int(pb + priv.max())
    bt = np.full((batch, width), -1, dtype=np.int32)
    cursor = 0
    for g in range(num_groups):
        shared = perm[cursor : cursor + pb]
        cursor += pb
        for j in range(group_size):
            i = g * group_size + j
            bt[i, :pb] = shared
            bt[i, pb : pb + priv[i]] = perm[cursor : cursor + priv[i]]
            cursor += int(priv[i])
    ctx = (prefix_len + gen_lens).astype(np.int32)
    return DecodeWorkload(
        name=name,
        num_blocks=num_blocks,
        block_size=block_size,
        num_kv_heads=num_kv_heads,
        num_q_heads=num_q_heads,
        head_dim=head_dim,
        context_lens=ctx,
        block_tables=bt,
        scale=1.0 / np.sqrt(head_dim),
        group_size=group_size,
        prefix_len=prefix_len,
    )


# ---------------------------------------------------------------------------
# The five workloads the path is measured and checked on.

def append_gather_workload(seqs: int = 32, max_len: int = 512, num_blocks: int = 2048) -> DecodeWorkload:
    """1 layer, 8 KV heads x 128, bf16, block 16, lengths U{1..512}, 2048-block pool.

    Lengths are the cached lengths before the append; one more token is appended
    per sequence, so ``context_lens = cached + 1``.
    """
    name = "append_gather"
    cached = randint(stream_key(name, "lens"), seqs, 1, max_len)
    return make_decode_workload(
        name,
        batch=seqs,
        num_kv_heads=8,
        num_q_heads=8,
        head_dim=128,
        block_size=16,
        context_lens=cached + 1,
        num_blocks=num_blocks,
    )


def qwen25_05b_workload(batch: int = 128) -> DecodeWorkload:
    """Qwen2.5-0.5B decode layer: 14 q / 2 kv heads, d=64, block 16, L U{256..2048}."""
    name = "qwen2.5-0.5b"
    lens = randint(stream_key(name, "lens"), batch, 256, 2048)
    return make_decode_workload(
        name, batch=batch, num_kv_heads=2, num_q_heads=14, head_dim=64, block_size=16, context_lens=lens
    )


def qwen3_4b_workload(batch: int = 64, context: int | None = 4096) -> DecodeWorkload:
    """Qwen3-4B decode layer: 32 q / 8 kv heads, d=128, block 16.

    ``context=4096`` is the fixed-length headline shape (4095 cached + 1 new);
    ``context=None`` draws lengths U{1024..8192}.
    """
    name = "qwen3-4b" if context is not None else "qwen3-4b-var"
    if context is None:
        lens = randint(stream_key(name, "lens"), batch, 1024, 8192)
    else:
        lens = np.full(batch, context, dtype=np.int64)
    return make_decode_workload(
        name, batch=batch, num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16, context_lens=lens
    )


def qwen25_7b_group_workload(num_groups: int = 32, group_size: int = 8, prefix_len: int = 1024,
                             max_gen: int = 3072) -> DecodeWorkload:
    """Qwen2.5-7B rollout groups: 28 q / 4 kv heads, d=128, shared 1024-token prompt."""
    name = "qwen2.5-7b-groups"
    gen = randint(stream_key(name, "gen"), num_groups * group_size, 0, max_gen) + 1
    return make_group_workload(
        name,
        num_groups=num_groups,
        group_size=group_size,
        prefix_len=prefix_len,
        gen_lens=gen,
        num_kv_heads=4,
        num_q_heads=28,
        head_dim=128,
        block_size=16,
    )


def deepseek_v3_mla_workload(batch: int = 32, context: int = 4096) -> DecodeWorkload:
    """DeepSeek-V3 MLA decode: 128 heads over one 576-wide latent entry, block 64."""
    name = "deepseek-v3-mla"
    lens = np.full(batch, context, dtype=np.int64)
    w = make_decode_workload(
        name, batch=batch, num_kv_heads=1, num_q_heads=128, head_dim=576, block_size=64, context_lens=lens,
        scale=1.0 / np.sqrt(192.0),
    )
    w.extras["kv_lora_rank"] = 512
    w.extras["rope_dim"] = 64
    return w
