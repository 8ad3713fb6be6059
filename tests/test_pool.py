"""KV pool lifecycle (CPU): sleep releases every layer's memory and the prefix
index, wake_up(tags) restores the pool as the engine drives it
(wavelet/inference/engine.py:858-873, scheduler.py:3201-3206)."""

import numpy as np
import pytest

from wavelet_amd import KVPool


def _pool(**kw):
    return KVPool(3, 64, 16, 2, 64, device="cpu", **kw)


def test_sleep_releases_memory_and_wake_restores_zeroed():
    pool = _pool()
    for c in pool.layers:
        c.k.fill_(1)
    assert pool.nbytes == 3 * 2 * 64 * 2 * 64 * 16 * 2
    pool.sleep()
    assert pool.asleep and all(c.k is None and c.v is None for c in pool.layers)
    with pytest.raises(RuntimeError, match="asleep"):
        pool.layers[0].descriptor()
    pool.wake_up(tags=["weights"])  # weights only: the KV pool stays released
    assert pool.asleep
    pool.wake_up(tags=["kv_cache"])
    assert not pool.asleep and all(int(c.k.abs().sum()) == 0 for c in pool.layers)
    pool.layers[0].descriptor()


def test_fp8_and_mla_pools_sleep_and_wake():
    pool = _pool(kv_dtype="fp8_e4m3")
    pool.sleep()
    assert all(c.k_scale is None for c in pool.layers)
    pool.wake_up()
    assert pool.layers[0].k_scale is not None and pool.layers[0].k.dtype.itemsize == 1
    mla = KVPool(2, 8, 64, mla=True, device="cpu")
    assert mla.nbytes == 2 * 8 * 64 * 576 * 2
    mla.sleep()
    assert mla.layers[0].latent is None
    mla.wake_up(["kv_cache", "weights"])
    assert tuple(mla.layers[0].latent.shape) == (8, 64, 576)


def test_sleep_resets_prefix_cache_and_refuses_live_sequences():
    pool = _pool()
    m = pool.blocks
    m.allocate("a", np.arange(40), cache_salt="v1")
    with pytest.raises(RuntimeError, match="still hold"):
        pool.sleep()
    assert not pool.asleep
    m.free("a")
    pool.sleep()
    # the prompt's full blocks are no longer matchable after wake (cache discarded)
    pool.wake_up()
    assert m.allocate("b", np.arange(40), cache_salt="v1") == 0
    assert "vllm:kv_cache_usage_perc" in pool.metrics_text()
    with pytest.raises(ValueError):
        pool.wake_up(tags=["bogus"])
    with pytest.raises(ValueError):
        pool.sleep(level=3)


# -- sizing from the engine's knobs (engine.py:790-813, configs/config.py:1003-1010) --------------------

GiB = 1 << 30


def _mem(free, total):
    return lambda: (free, total)


def test_from_engine_config_derives_num_gpu_blocks_from_the_utilization_share():
    # 4 layers x 2 kv heads x d=64 x block 16, bf16: 2 * 16 * 2 * 64 * 2 = 8 KiB per layer, 32 KiB per block id
    kw = dict(num_layers=4, num_kv_heads=2, head_dim=64, block_size=16, device="cpu")
    pool = KVPool.from_engine_config(gpu_memory_utilization=0.5, reserve_bytes=1 << 20, non_kv_bytes=3 << 20,
                                     mem_get_info=_mem(64 << 20, 64 << 20), **kw)
    per_block = 4 * 2 * 16 * 2 * 64 * 2
    assert pool.num_blocks == ((32 << 20) - (1 << 20) - (3 << 20)) // per_block == 896
    assert pool.nbytes == pool.num_blocks * per_block <= (32 << 20) - (4 << 20)
    assert f'num_gpu_blocks="{pool.num_blocks}"' in pool.metrics_text()
    assert pool.max_model_len is None and pool.blocks.max_blocks_per_seq is None
    # the default utilization is the reference's 0.35
    p35 = KVPool.from_engine_config(reserve_bytes=0, mem_get_info=_mem(64 << 20, 64 << 20), **kw)
    assert p35.num_blocks == int(0.35 * (64 << 20)) // per_block


def test_from_engine_config_fp8_and_mla_block_bytes():
    from wavelet_amd.pool import block_bytes

    assert block_bytes(36, 16, 8, 128) == 36 * 2 * 16 * 8 * 128 * 2
    assert block_bytes(28, 16, 4, 128, "fp8_e4m3") == 28 * (2 * 16 * 4 * 128 + 2 * 4 * 4)
    assert block_bytes(8, 64, mla=True) == 8 * 64 * 576 * 2
    pool = KVPool.from_engine_config(num_layers=2, num_kv_heads=1, head_dim=64, kv_dtype="fp8_e4m3", block_size=16,
                                     gpu_memory_utilization=1.0, reserve_bytes=0,
                                     mem_get_info=_mem(1 << 20, 1 << 20), device="cpu")
    assert pool.num_blocks == (1 << 20) // (2 * (2 * 16 * 64 + 8)) and pool.layers[0].k_scale is not None
    mla = KVPool.from_engine_config(num_layers=2, block_size=64, mla=True, gpu_memory_utilization=1.0,
                                    reserve_bytes=0, mem_get_info=_mem(1 << 22, 1 << 22), device="cpu")
    assert mla.num_blocks == (1 << 22) // (2 * 64 * 576 * 2)


def test_from_engine_config_refuses_what_the_engine_refuses():
    kw = dict(num_layers=4, num_kv_heads=2, head_dim=64, block_size=16, device="cpu", reserve_bytes=0)
    with pytest.raises(ValueError, match="gpu_memory_utilization"):
        KVPool.from_engine_config(gpu_memory_utilization=0.0, mem_get_info=_mem(GiB, GiB), **kw)
    with pytest.raises(ValueError, match="gpu_memory_utilization"):
        KVPool.from_engine_config(gpu_memory_utilization=1.5, mem_get_info=_mem(GiB, GiB), **kw)
    # the share must be free now (another process holds most of the device)
    with pytest.raises(ValueError, match="free device memory"):
        KVPool.from_engine_config(gpu_memory_utilization=0.5, mem_get_info=_mem(GiB // 4, GiB), **kw)
    # weights take the whole share
    with pytest.raises(ValueError, match="no memory for KV blocks"):
        KVPool.from_engine_config(gpu_memory_utilization=0.5, non_kv_bytes=GiB // 2, mem_get_info=_mem(GiB, GiB),
                                  **kw)
    # one max_model_len sequence must fit: 1 MiB / 32 KiB = 32 blocks = 512 tokens
    small = _mem(2 << 20, 2 << 20)
    assert KVPool.from_engine_config(gpu_memory_utilization=0.5, max_model_len=512, mem_get_info=small,
                                     **kw).num_blocks == 32
    with pytest.raises(ValueError, match="max_model_len 513"):
        KVPool.from_engine_config(gpu_memory_utilization=0.5, max_model_len=513, mem_get_info=small, **kw)


def test_max_model_len_bounds_tables_and_admission():
    pool = KVPool.from_engine_config(num_layers=1, num_kv_heads=2, head_dim=64, block_size=16,
                                     gpu_memory_utilization=1.0, reserve_bytes=0, max_model_len=40,
                                     mem_get_info=_mem(1 << 20, 1 << 20), device="cpu")
    m = pool.blocks
    assert pool.max_model_len == 40 and m.max_blocks_per_seq == 3
    with pytest.raises(ValueError, match="longer than max_model_len"):
        m.allocate("long", np.arange(41))
    m.allocate("a", np.arange(38))
    m.allocate("b", np.arange(5))
    m.append_slots(["a", "b"])  # a: 39 tokens
    m.append_slots(["a", "b"])  # a: 40 tokens, at the limit
    before = (m.seq_len("a"), m.seq_len("b"), m.num_free_blocks)
    with pytest.raises(ValueError, match="max_model_len is 40"):
        m.append_slots(["b", "a"])
    assert (m.seq_len("a"), m.seq_len("b"), m.num_free_blocks) == before  # refused before any change
    bt, lens = m.tables(["a", "b"])
    assert bt.shape == (2, 3) and lens.tolist() == [40, 7]
    with pytest.raises(ValueError, match="exceeds the pool"):
        KVPool(1, 2, 16, 2, 64, max_model_len=33, device="cpu")


def test_read_policy_descriptors_and_step_choice():
    """Each cache carries one descriptor per read policy (flags 0 / WKV_CACHE_SHARED_BLOCKS);
    a pool's layers default to the shared-safe policy, a step over sequences that share no
    block chooses the streaming one, and the default cannot be changed after construction
    (the descriptors are built once)."""
    from wavelet_amd import PagedKVCache, _lib

    pool = KVPool(2, 64, 16, 2, 64, device="cpu")
    c = pool.layers[0]
    assert c.shared_blocks and c.descriptor().flags == _lib.CACHE_SHARED_BLOCKS
    assert c.descriptor(False).flags == 0 and c.descriptor(True).flags == _lib.CACHE_SHARED_BLOCKS
    assert c.descriptor(False).k == c.descriptor(True).k == c.k.data_ptr()
    with pytest.raises(AttributeError):
        c.shared_blocks = False
    plain = PagedKVCache(8, 16, 2, 64, device="cpu")
    assert not plain.shared_blocks and plain.descriptor().flags == 0
    m = pool.blocks
    m.allocate("a", np.arange(20))
    m.allocate("b", np.arange(33) + 50)
    assert not pool.decode_shares_blocks(["a", "b"])
    m.fork("a", "a2")
    assert pool.decode_shares_blocks(["b", "a2"])
    for s in ("a", "a2", "b"):
        m.free(s)
    pool.sleep()
    with pytest.raises(RuntimeError, match="asleep"):
        c.descriptor(False)
