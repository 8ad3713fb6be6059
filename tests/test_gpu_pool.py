"""KV pool sleep/wake on the GPU: the device memory is returned and the pool
works again after wake_up (append + decode through the block manager)."""

import math

import numpy as np
import pytest
import torch

from wavelet_amd import KVPool, paged_decode_gqa

pytestmark = pytest.mark.gpu


def test_sleep_returns_device_memory_and_wake_restores_a_working_pool(cuda):
    pool = KVPool(4, 512, 16, 8, 128, device=cuda)
    torch.cuda.synchronize()
    awake = torch.cuda.memory_allocated(cuda)
    pool.sleep()
    torch.cuda.synchronize()
    asleep = torch.cuda.memory_allocated(cuda)
    assert awake - asleep >= pool.nbytes, (awake, asleep, pool.nbytes)
    pool.wake_up(tags=["weights"])
    assert pool.asleep
    pool.wake_up(tags=["kv_cache"])
    assert torch.cuda.memory_allocated(cuda) - asleep >= pool.nbytes
    # a prompt and one decode step through the woken pool
    m = pool.blocks
    m.allocate("s", np.arange(40))
    bt, lens = m.tables(["s"])
    pos = np.arange(40)
    slots = torch.from_numpy(np.array(m.blocks_of("s"), np.int64)[pos // 16] * 16 + pos % 16).to(cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(3)
    k = torch.randn((40, 8, 128), generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn((40, 8, 128), generator=g, device=cuda).to(torch.bfloat16)
    for c in pool.layers:
        c.append(k, v, slots)
    q = torch.randn((1, 32, 128), generator=g, device=cuda).to(torch.bfloat16)
    out = paged_decode_gqa(q, pool.layers[2], torch.from_numpy(bt).to(cuda), torch.from_numpy(lens).to(cuda),
                           1 / math.sqrt(128))
    # reference: plain softmax attention over the 40 tokens (float32)
    qf = q.float()[0].view(8, 4, 128)
    s = torch.einsum("hgd,thd->hgt", qf, k.float()) / math.sqrt(128)
    ref = torch.einsum("hgt,thd->hgd", torch.softmax(s, -1), v.float()).reshape(32, 128)
    torch.testing.assert_close(out.float()[0], ref, atol=2e-2, rtol=1e-2)
