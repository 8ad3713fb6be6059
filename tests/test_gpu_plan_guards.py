"""Plan construction refuses what would make a launch read out of bounds, and a plan
kept across a pool's sleep / wake_up refuses to launch on released memory.

Every check here happens on the host before any launch; the sleep / wake tests
replace the plan's library handle with one that fails the test on any call, so a
broken guard shows up as that failure and never as a kernel on freed memory.
"""

import numpy as np
import pytest
import torch

from wavelet_amd import KVPool, MLALatentCache, PagedKVCache, synth
from wavelet_amd.plan import DecodeStep, MLADecodeStep, PrefillStep

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


class _NoLaunch:
    """Stands in for the ctypes library: any entry point fails the test."""

    def __getattr__(self, name):
        def fail(*_a, **_k):
            raise AssertionError(f"{name} was called: the plan launched on a released cache")

        return fail


def _gqa_inputs(cuda, layers=2, batch=4, hq=8, hkv=2, d=64, bs=16):
    w = synth.make_decode_workload("guards", batch=batch, num_kv_heads=hkv, num_q_heads=hq, head_dim=d,
                                   block_size=bs, context_lens=np.array([5, 17, 40, 64][:batch]))
    q = [torch.zeros((batch, hq, d), dtype=BF16, device=cuda) for _ in range(layers)]
    k = [torch.zeros((batch, hkv, d), dtype=BF16, device=cuda) for _ in range(layers)]
    v = [torch.zeros((batch, hkv, d), dtype=BF16, device=cuda) for _ in range(layers)]
    o = [torch.zeros((batch, hq, d), dtype=BF16, device=cuda) for _ in range(layers)]
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    slots = torch.from_numpy(w.new_token_slots()).to(cuda)
    return w, q, k, v, o, bt, sl, slots


def test_decode_plan_refuses_host_or_short_slot_mappings_and_strided_tables(cuda):
    w, q, k, v, o, bt, sl, slots = _gqa_inputs(cuda)
    caches = [PagedKVCache(w.num_blocks, 16, 2, 64, device=cuda) for _ in range(2)]
    args = (caches, q, k, v, o, bt, sl)
    with pytest.raises(ValueError, match="slot_mapping is on cpu"):
        DecodeStep(*args, slots.cpu(), w.scale, 64)
    with pytest.raises(ValueError, match="one slot per sequence"):
        DecodeStep(*args, slots[:3].contiguous(), w.scale, 64)
    wide = torch.zeros((w.batch, 2 * bt.shape[1]), dtype=torch.int32, device=cuda)
    wide[:, ::2] = bt
    with pytest.raises(ValueError, match="contiguous rows"):
        DecodeStep(caches, q, k, v, o, wide[:, ::2], sl, slots, w.scale, 64)
    sl2 = torch.zeros(2 * w.batch, dtype=torch.int32, device=cuda)
    sl2[::2] = sl
    with pytest.raises(ValueError, match="contiguous seq_lens"):
        DecodeStep(caches, q, k, v, o, bt, sl2[::2], slots, w.scale, 64)
    with pytest.raises(ValueError, match="one tensor per layer"):
        DecodeStep(caches, q[:1], k, v, o, bt, sl, slots, w.scale, 64)
    DecodeStep(*args, slots, w.scale, 64)  # the valid plan builds


def test_mla_and_prefill_plans_refuse_host_or_short_slot_mappings(cuda):
    B, H, R, P, BS = 3, 16, 512, 64, 64
    w = synth.make_decode_workload("mlaguards", batch=B, num_kv_heads=1, num_q_heads=H, head_dim=R + P,
                                   block_size=BS, context_lens=np.array([1, 70, 130]))
    caches = [MLALatentCache(w.num_blocks, BS, R, P, device=cuda)]
    qn = [torch.zeros((B, H, R), dtype=BF16, device=cuda)]
    qp = [torch.zeros((B, H, P), dtype=BF16, device=cuda)]
    kc = [torch.zeros((B, R), dtype=BF16, device=cuda)]
    kp = [torch.zeros((B, P), dtype=BF16, device=cuda)]
    o = [torch.zeros((B, H, R), dtype=BF16, device=cuda)]
    bt = torch.from_numpy(w.block_tables).to(cuda)
    sl = torch.from_numpy(w.context_lens).to(cuda)
    slots = torch.from_numpy(w.new_token_slots()).to(cuda)
    with pytest.raises(ValueError, match="slot_mapping is on cpu"):
        MLADecodeStep(caches, qn, qp, kc, kp, o, bt, sl, slots.cpu(), 0.1, 130)
    with pytest.raises(ValueError, match="one slot per sequence"):
        MLADecodeStep(caches, qn, qp, kc, kp, o, bt, sl, slots[:2].contiguous(), 0.1, 130)
    MLADecodeStep(caches, qn, qp, kc, kp, o, bt, sl, slots, 0.1, 130)

    w2, *_ = _gqa_inputs(cuda)
    T = 8
    pc = [PagedKVCache(w2.num_blocks, 16, 2, 64, device=cuda)]
    cu = torch.tensor([0, 2, 4, 6, 8], dtype=torch.int32, device=cuda)
    pq = [torch.zeros((T, 8, 64), dtype=BF16, device=cuda)]
    pk = [torch.zeros((T, 2, 64), dtype=BF16, device=cuda)]
    po = [torch.zeros((T, 8, 64), dtype=BF16, device=cuda)]
    pslots = torch.arange(T, dtype=torch.int64, device=cuda)
    bt2, sl2 = torch.from_numpy(w2.block_tables).to(cuda), torch.from_numpy(w2.context_lens).to(cuda)
    with pytest.raises(ValueError, match="slot_mapping is on cpu"):
        PrefillStep(pc, pq, pk, pk, po, bt2, sl2, cu, pslots.cpu(), 0.1, 2, 64)
    with pytest.raises(ValueError, match="cu_seqlens_q is on cpu"):
        PrefillStep(pc, pq, pk, pk, po, bt2, sl2, cu.cpu(), pslots, 0.1, 2, 64)
    PrefillStep(pc, pq, pk, pk, po, bt2, sl2, cu, pslots, 0.1, 2, 64)


@pytest.mark.parametrize("kind", ["decode", "prefill", "mla"])
def test_plans_refuse_to_launch_after_sleep_and_after_wake(cuda, kind):
    if kind == "mla":
        B, H, R, P, BS = 3, 16, 512, 64, 64
        w = synth.make_decode_workload("mlasleep", batch=B, num_kv_heads=1, num_q_heads=H, head_dim=R + P,
                                       block_size=BS, context_lens=np.array([1, 70, 130]))
        pool = KVPool(2, w.num_blocks, BS, mla=True, device=cuda)
        z = lambda *s: [torch.zeros(s, dtype=BF16, device=cuda) for _ in range(2)]  # noqa: E731
        step = MLADecodeStep(pool.layers, z(B, H, R), z(B, H, P), z(B, R), z(B, P), z(B, H, R),
                             torch.from_numpy(w.block_tables).to(cuda), torch.from_numpy(w.context_lens).to(cuda),
                             torch.from_numpy(w.new_token_slots()).to(cuda), 0.1, 130)
    else:
        w, q, k, v, o, bt, sl, slots = _gqa_inputs(cuda)
        pool = KVPool(2, w.num_blocks, 16, 2, 64, device=cuda)
        if kind == "decode":
            step = DecodeStep(pool.layers, q, k, v, o, bt, sl, slots, w.scale, 64, order_by_length=True)
        else:
            cu = torch.arange(0, 5, dtype=torch.int32, device=cuda)
            step = PrefillStep(pool.layers, q, k, v, o, bt, sl, cu, slots, w.scale, 1, 64)
    step.run()  # a live plan launches
    torch.cuda.synchronize()
    step.lib = _NoLaunch()
    if hasattr(step, "calls") and kind == "decode":
        for c in step.calls:
            c.append_fn = _NoLaunch().wkv_append
    elif kind == "prefill":
        step.calls = [(_NoLaunch().wkv_append, *c[1:]) for c in step.calls]
    pool.sleep()
    with pytest.raises(RuntimeError, match="asleep"):
        step.run()
    for layer in range(2):
        for op in ("append", "attend", "step_layer"):
            with pytest.raises(RuntimeError, match="asleep"):
                getattr(step, op)(layer)
    pool.wake_up()
    with pytest.raises(RuntimeError, match="re-allocated"):
        step.run()
    with pytest.raises(RuntimeError, match="re-allocated"):
        step.step_layer(1)
