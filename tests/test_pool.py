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
