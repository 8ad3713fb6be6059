"""Host-side block management (CPU only): sharing, copy-on-write, salted prefix reuse, metrics."""

import re

import numpy as np
import pytest

from wavelet_amd import BlockManager


def test_capacity_and_metrics_lines_match_the_scraped_format():
    m = BlockManager(2048, 16)
    # tests/test_adaptive_concurrency.py:211-222 in the reference: 16 x 2048 = 32768 tokens
    assert m.capacity_tokens == 32_768
    text = m.metrics_text()
    assert 'vllm:cache_config_info{block_size="16",num_gpu_blocks="2048"} 1' in text
    labels = dict(re.findall(r'(\w+)="([^"]*)"', text))
    assert int(labels["num_gpu_blocks"]) * int(labels["block_size"]) == 32_768
    m.allocate("a", np.arange(100))
    usage = float(re.search(r"vllm:kv_cache_usage_perc (\S+)", m.metrics_text()).group(1))
    assert usage == pytest.approx(7 / 2048, abs=1e-6)


def test_group_shares_whole_prompt_blocks_without_copies():
    m = BlockManager(256, 16)
    m.allocate("g0", np.arange(1024))  # 64 full blocks
    for j in range(1, 8):
        m.fork("g0", f"g{j}")
    prompt = m.blocks_of("g0")
    assert all(m.ref_count(b) == 8 for b in prompt)
    slots, cow = m.append_slots([f"g{j}" for j in range(8)])
    assert cow == []  # the prompt ends on a block boundary: every member opens a private block
    blocks = slots // 16
    assert len(set(blocks.tolist())) == 8 and not set(blocks.tolist()) & set(prompt)
    assert np.all(slots % 16 == 0)
    bt, lens = m.tables([f"g{j}" for j in range(8)])
    assert np.all(lens == 1025) and np.all(bt[:, :64] == np.array(prompt))


def test_partial_shared_block_is_copied_on_first_write():
    m = BlockManager(64, 16)
    m.allocate("p", np.arange(40))  # 2 full blocks + 8 tokens in a third
    m.fork("p", "c1")
    m.fork("p", "c2")
    last = m.blocks_of("p")[2]
    assert m.ref_count(last) == 3
    slots, cow = m.append_slots(["c1", "c2", "p"])
    # c1 and c2 each copy the shared partial block; p then owns the original alone
    assert [src for src, _ in cow] == [last, last]
    assert slots[2] == last * 16 + 8 and m.ref_count(last) == 1
    for (src, dst), s in zip(cow, slots[:2]):
        assert s == dst * 16 + 8 and m.ref_count(dst) == 1
    assert m.blocks_of("c1")[:2] == m.blocks_of("p")[:2]


def test_share_prefix_takes_the_first_blocks():
    m = BlockManager(64, 16)
    m.allocate("src", np.arange(50))
    m.share_prefix("src", ["x", "y"], 2)
    assert m.blocks_of("x") == m.blocks_of("src")[:2] and m.seq_len("y") == 32
    with pytest.raises(ValueError):
        m.share_prefix("src", ["z"], 9)


def test_prefix_cache_is_keyed_by_salt_and_cleared_by_reset():
    m = BlockManager(64, 16)
    prompt = np.arange(70)
    assert m.allocate("a", prompt, cache_salt="step-1") == 0
    assert m.allocate("b", prompt, cache_salt="step-1") == 64  # 4 full blocks reused
    assert m.blocks_of("b")[:4] == m.blocks_of("a")[:4]
    assert m.allocate("c", prompt, cache_salt="step-2") == 0  # another policy step: no sharing
    assert m.allocate("d", prompt) == 0  # no salt differs from any salt
    m.free("a")
    m.free("b")
    assert m.allocate("e", prompt, cache_salt="step-1") == 64  # released blocks stay matchable
    m.free("e")
    m.reset_prefix_cache()
    assert m.allocate("f", prompt, cache_salt="step-1") == 0


def test_free_and_exhaustion():
    m = BlockManager(4, 16)
    m.allocate("a", np.arange(48))
    with pytest.raises(MemoryError):
        m.allocate("b", np.arange(1000, 1040))  # no prefix in common: needs 3 fresh blocks
    assert m.num_free_blocks == 1  # the failed allocation gave its blocks back
    m.free("a")
    assert m.num_free_blocks == 4 and m.usage == 0.0
    m2 = BlockManager(2, 16, enable_prefix_caching=False)
    m2.allocate("a", np.arange(32))
    with pytest.raises(MemoryError):
        m2.append_slots(["a"])


def test_cached_blocks_are_evicted_lru_when_space_runs_out():
    m = BlockManager(4, 16)
    m.allocate("a", np.arange(32), cache_salt="s")  # 2 indexed full blocks
    m.free("a")
    assert m.num_free_blocks == 4
    m.allocate("b", np.arange(100, 164))  # needs all 4: evicts the cached ones
    m.free("b")
    assert m.allocate("c", np.arange(32), cache_salt="s") == 0


def test_validate_group_prefix_accepts_true_claims_and_names_false_ones():
    from wavelet_amd import synth, validate_group_prefix

    w = synth.make_group_workload("vgp", num_groups=3, group_size=4, prefix_len=64,
                                  gen_lens=np.array([1, 5, 17, 40, 20, 21, 22, 23, 9, 30, 2, 16]), num_kv_heads=1,
                                  num_q_heads=1, head_dim=64, block_size=16)
    bt, lens = w.block_tables, w.context_lens
    ok = np.full(3, 64, np.int32)
    validate_group_prefix(bt, lens, ok, 4, 16)
    validate_group_prefix(bt, lens, ok, 4, 16, appending=True)
    validate_group_prefix(bt, lens, np.array([70, 79, 0], np.int32), 4, 16)  # 70 // 16 = 4 blocks: still shared
    # a claim reaching into the members' private blocks (group 1's members all hold 84+ tokens)
    with pytest.raises(ValueError, match="group 1: prefix_lens 80 claims block 4 shared"):
        validate_group_prefix(bt, lens, np.array([64, 80, 64], np.int32), 4, 16)
    # a member whose prompt block differs inside a true-looking claim
    bad = bt.copy()
    bad[6, 2] = bt[0, 2]
    with pytest.raises(ValueError, match="member 6 holds block"):
        validate_group_prefix(bad, lens, ok, 4, 16)
    validate_group_prefix(bad, lens, np.array([64, 32, 64], np.int32), 4, 16)  # claim stops before block 2
    # ragged last group (batch 10 in groups of 4) and a claim past every member's length
    validate_group_prefix(bt[:10], lens[:10], np.array([64, 64, 64], np.int32), 4, 16)
    short = lens.copy()
    short[:4] = [65, 65, 65, 65]
    with pytest.raises(ValueError, match="claims block 4"):
        validate_group_prefix(bt, lens + 100, np.array([1000, 64, 64], np.int32), 4, 16)
    validate_group_prefix(bt, short, np.array([1000, 64, 64], np.int32), 4, 16)  # cut to the shortest member
    with pytest.raises(ValueError, match="one entry per group"):
        validate_group_prefix(bt, lens, ok[:2], 4, 16)


def _state(m, ids):
    return ([m.blocks_of(s) for s in ids], [m.seq_len(s) for s in ids], m.num_free_blocks,
            [m.ref_count(b) for b in range(m.num_blocks)])


def test_multi_token_append_slots_follow_each_table_and_copy_once():
    m = BlockManager(64, 16)
    m.allocate("p", np.arange(40))  # the third block is partly filled
    m.fork("p", "c")
    last = m.blocks_of("p")[2]
    slots, cow = m.append_slots(["c", "p"], 20)  # 8 + 12 tokens: fills the third block, opens a fourth
    assert cow == [(last, m.blocks_of("c")[2])]
    for i, sid in enumerate(["c", "p"]):
        table = np.asarray(m.blocks_of(sid), np.int64)
        pos = np.arange(40, 60)
        np.testing.assert_array_equal(slots[i * 20:(i + 1) * 20], table[pos // 16] * 16 + pos % 16)
        assert m.seq_len(sid) == 60 and len(table) == 4
    assert m.ref_count(last) == 1 and m.blocks_of("p")[2] == last
    assert m.blocks_needed(["c", "p"], 0) == 0


def test_append_slots_changes_nothing_when_the_step_cannot_be_taken():
    m = BlockManager(8, 16, max_model_len=64)
    m.allocate("a", np.arange(30))
    m.fork("a", "b")
    m.allocate("c", np.arange(60))
    before = _state(m, ["a", "b", "c"])
    with pytest.raises(ValueError, match="max_model_len"):
        m.append_slots(["a", "b", "c"], 5)  # c would reach 65
    assert _state(m, ["a", "b", "c"]) == before
    # a and b need a copy of their shared partial block plus fresh ones: more than the free pool
    assert m.blocks_needed(["a", "b"], 30) > m.num_free_blocks
    with pytest.raises(MemoryError):
        m.append_slots(["a", "b"], 30)
    assert _state(m, ["a", "b", "c"]) == before
    with pytest.raises(ValueError, match="twice"):
        m.append_slots(["a", "a"])
    assert _state(m, ["a", "b", "c"]) == before
    # the same step within the limits goes through
    slots, cow = m.append_slots(["a", "b"], 2)
    assert len(slots) == 4 and len(cow) == 1


def test_blocks_needed_counts_exactly_what_append_slots_takes():
    rng = np.random.default_rng(5)
    for trial in range(30):
        m = BlockManager(400, 16)
        ids = []
        for g in range(4):
            n = int(rng.integers(1, 60))
            m.allocate(f"g{g}", np.arange(n) + 1000 * trial + 100 * g)
            ids.append(f"g{g}")
            for j in range(int(rng.integers(0, 4))):
                m.fork(f"g{g}", f"g{g}.{j}")
                ids.append(f"g{g}.{j}")
        rng.shuffle(ids)
        n = int(rng.integers(1, 40))
        need = m.blocks_needed(ids, n)
        free = m.num_free_blocks
        m.append_slots(ids, n)
        assert free - m.num_free_blocks == need


def test_any_shared_follows_reference_counts():
    m = BlockManager(64, 16)
    m.allocate("a", np.arange(20))
    m.allocate("x", np.arange(40) + 99)
    assert not m.any_shared(["a", "x"])
    m.fork("a", "b")
    assert m.any_shared(["a"]) and m.any_shared(["b", "x"])
    m.append_slots(["a", "b"], 20)  # b copies the partial block; the full first block stays shared
    assert m.any_shared(["a", "b"])
    m.free("b")
    assert not m.any_shared(["a", "x"])
