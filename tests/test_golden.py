"""Golden fixtures and the seeded generator (CPU only).

The generator must reproduce the committed input checksums byte for byte
(the GPU host regenerates the same inputs), and the oracle must reproduce the
committed expected outputs.
"""

import json

import numpy as np
import torch

from golden import make_golden as mg
from oracle import paged
from wavelet_amd import synth


def test_generator_reproduces_committed_input_checksums(golden_dir):
    expected = json.loads((golden_dir / "checksums.json").read_text())
    assert mg.checksums() == expected


def test_bf16_rounding_matches_torch():
    x = synth.normal(synth.stream_key("synth", "bf16"), 1 << 16) * 1e3
    x = np.concatenate([x, [np.inf, -np.inf, 0.0, -0.0, 1e-40, 3.4e38]])
    ref = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(synth.to_bf16_bits(x), ref)
    # NaN stays NaN (its payload and sign are a convention the generator never relies on)
    nan_bits = int(synth.to_bf16_bits(np.array([np.nan]))[0])
    assert (nan_bits & 0x7F80) == 0x7F80 and (nan_bits & 0x7F) != 0


def test_generator_distributions():
    z = synth.normal(synth.stream_key("synth", "moments"), 200_000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    r = synth.randint(synth.stream_key("synth", "ints"), 100_000, 1, 512)
    assert r.min() == 1 and r.max() == 512 and abs(r.mean() - 256.5) < 3
    p = synth.permutation(synth.stream_key("synth", "perm"), 2048)
    assert np.array_equal(np.sort(p), np.arange(2048))


def test_workload_shapes_follow_the_configs():
    w = synth.append_gather_workload()
    assert (w.batch, w.num_kv_heads, w.head_dim, w.block_size, w.num_blocks) == (32, 8, 128, 16, 2048)
    assert w.context_lens.min() >= 2 and w.context_lens.max() <= 513
    w = synth.qwen3_4b_workload()
    assert (w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim) == (64, 32, 8, 128)
    assert np.all(w.context_lens == 4096) and w.num_blocks == 64 * 256
    w = synth.qwen25_7b_group_workload()
    assert w.batch == 256 and w.group_size == 8 and w.prefix_len == 1024
    # members of a group share the prompt's physical blocks, private blocks are disjoint
    bt = w.block_tables
    assert np.array_equal(bt[0, :64], bt[7, :64]) and not np.array_equal(bt[0, :64], bt[8, :64])
    used = np.concatenate([bt[i, :(int(w.context_lens[i]) + 15) // 16] for i in range(w.batch)])
    assert len(np.unique(used)) == 32 * 64 + sum((int(L) - 1024 + 15) // 16 for L in w.context_lens)


def test_oracle_reproduces_append_gather_digests(golden_dir):
    assert mg.append_gather() == json.loads((golden_dir / "outputs.json").read_text())["append_gather"]


def test_oracle_reproduces_fp8_block(golden_dir):
    g = np.load(golden_dir / "fp8_block.npz")
    kc, vc = paged.empty_cache(4, 16, 1, 128, dtype=np.uint8)
    ks = np.zeros((4, 1), np.float32)
    vs = np.zeros((4, 1), np.float32)
    for i in range(4):
        paged.append_fp8(kc, vc, ks, vs, g[f"k{i}"], g[f"v{i}"], g[f"slots{i}"])
    np.testing.assert_array_equal(kc, g["k_cache"])
    np.testing.assert_array_equal(vc, g["v_cache"])
    np.testing.assert_array_equal(ks, g["k_scale"])
    np.testing.assert_array_equal(vs, g["v_scale"])


def test_oracle_reproduces_gqa_decode(golden_dir):
    w, k, v, q = mg.gqa_decode_case()
    assert synth.sha256_of(w.block_tables, w.context_lens, k, v, q) == \
        json.loads((golden_dir / "outputs.json").read_text())["gqa_decode_inputs"]
    out = paged.decode_gqa(paged.bf16_to_f32(q), paged.bf16_to_f32(k), paged.bf16_to_f32(v), w.block_tables,
                           w.context_lens, w.scale)
    np.testing.assert_allclose(out, np.load(golden_dir / "gqa_decode.npz")["out"], rtol=1e-12, atol=1e-14)


def test_ignore_slot_fixture_holds_the_reference_answer(golden_dir):
    g = np.load(golden_dir / "ignore_slot.npz")
    out = paged.decode_gqa(g["q"], g["k_logical"], g["v_logical"], g["block_tables"], g["context_lens"],
                           float(g["scale"]))
    np.testing.assert_allclose(out, g["expected"], rtol=1e-12, atol=1e-12)
    assert abs(g["expected"][0, 0, 0] - 2.0 / (1.0 + np.exp(-0.625))) < 1e-15
