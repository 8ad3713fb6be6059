"""The reference's attention call convention on the paged path, end to end.

The Qwen3 attention forward (transformers' own, the sequence the reference
patches at wavelet/kernels/patch.py:173-196) runs ``past_key_values.update``
then ``attention_interface(..., scaling=...)``. A two-layer Qwen3 model with
random bf16 weights runs a prompt in two chunks and six decode steps with a
``PagedCache`` on a ``KVPool`` and ``attn_implementation="wavelet_paged"``; the
reference is the same model with transformers' eager attention in fp32 and a
DynamicCache. Bar: at every step the paged logits are no further from the fp32
logits than 1.5 times the distance of transformers' own bf16 eager run (plus
0.005 absolute; measured on MI355X the two distances are alike, 0.017-0.028),
and the cache holds the model's rows where the block manager put them."""

import pytest
import torch

pytest.importorskip("transformers")

from transformers import DynamicCache, Qwen3Config, Qwen3ForCausalLM

from wavelet_amd import KVPool
from wavelet_amd.hf import PagedCache, register

pytestmark = pytest.mark.gpu

B, CHUNKS, DECODE = 3, (37, 20), 6


def _config():
    return Qwen3Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                       num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                       tie_word_embeddings=False)


def _run(model, cache, ids):
    """Logits of every step: the prompt chunks, then one token per step (teacher-forced)."""
    outs, pos = [], 0
    for n in CHUNKS:
        outs.append(model(ids[:, pos:pos + n], past_key_values=cache, use_cache=True).logits.float())
        pos += n
    for _ in range(DECODE):
        outs.append(model(ids[:, pos:pos + 1], past_key_values=cache, use_cache=True).logits.float())
        pos += 1
    return outs


@torch.no_grad()
def test_qwen3_steps_through_paged_cache(cuda):
    torch.manual_seed(1234)
    cfg = _config()
    ref32 = Qwen3ForCausalLM(cfg).to(device=cuda, dtype=torch.float32).eval()
    ref32.set_attn_implementation("eager")
    model = Qwen3ForCausalLM(cfg).to(device=cuda, dtype=torch.bfloat16).eval()
    model.load_state_dict({k: v.to(torch.bfloat16) for k, v in ref32.state_dict().items()})
    gen = torch.Generator(device="cpu").manual_seed(99)
    ids = torch.randint(0, cfg.vocab_size, (B, sum(CHUNKS) + DECODE), generator=gen).to(cuda)

    want = _run(ref32, DynamicCache(config=cfg), ids)
    model.set_attn_implementation("eager")
    eager16 = _run(model, DynamicCache(config=cfg), ids)

    pool = KVPool(num_layers=cfg.num_hidden_layers, num_blocks=64, block_size=16, num_kv_heads=2, head_dim=128,
                  device=cuda)
    seq_ids = [10, 11, 12]
    cache = PagedCache(pool, seq_ids)
    model.set_attn_implementation(register())
    got = _run(model, cache, ids)

    print("step  |paged-fp32|  |eager16-fp32|")
    for i, (g, e, w) in enumerate(zip(got, eager16, want)):
        assert torch.isfinite(g).all(), f"step {i}: non-finite logits"
        d_paged = (g - w).abs().max().item()
        d_eager = (e - w).abs().max().item()
        print(f"{i:4d}  {d_paged:.4f}  {d_eager:.4f}")
        assert d_paged <= 1.5 * d_eager + 0.005, f"step {i}: paged {d_paged:.4f} vs eager bf16 {d_eager:.4f}"

    total = sum(CHUNKS) + DECODE
    assert cache.get_seq_length() == total
    assert all(pool.blocks.seq_len(s) == total for s in seq_ids)
    # the cache rows sit where the block manager says: layer 0's K of sequence 11, token 40,
    # against a fresh eager run's cache (layer 0's K does not depend on the attention path)
    dyn = DynamicCache(config=cfg)
    model.set_attn_implementation("eager")
    model(ids[:, :total], past_key_values=dyn, use_cache=True)
    k_ref = dyn.layers[0].keys[1, :, 40]  # [Hkv, D]
    bt, sl = pool.blocks.tables([seq_ids[1]])
    k_all, _ = pool.layers[0].gather(torch.from_numpy(bt).to(cuda), torch.from_numpy(sl).to(cuda))
    torch.testing.assert_close(k_all[40].float(), k_ref.float(), atol=2e-2, rtol=2e-2)


@torch.no_grad()
def test_gpt_oss_sinks_through_paged_cache(cuda):
    """A model with learned attention sinks (transformers' GPT-OSS passes them as ``s_aux``), all
    layers full attention, random weights with non-zero sinks: prompt chunks and decode steps on
    the paged path (prefill and decode kernels with sinks) against the same model's eager fp32
    run, at the bar of the Qwen3 test above."""
    cfg_mod = pytest.importorskip("transformers.models.gpt_oss")
    cfg = cfg_mod.GptOssConfig(vocab_size=512, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                               num_attention_heads=8, num_key_value_heads=2, head_dim=64, num_local_experts=4,
                               num_experts_per_tok=2, max_position_embeddings=4096, sliding_window=128,
                               layer_types=["full_attention", "full_attention"], tie_word_embeddings=False)
    torch.manual_seed(4321)
    ref32 = cfg_mod.GptOssForCausalLM(cfg).to(device=cuda, dtype=torch.float32).eval()
    for layer in ref32.model.layers:
        layer.self_attn.sinks.normal_(mean=1.0, std=2.0)
    ref32.set_attn_implementation("eager")
    model = cfg_mod.GptOssForCausalLM(cfg).to(device=cuda, dtype=torch.bfloat16).eval()
    model.load_state_dict({k: v.to(torch.bfloat16) for k, v in ref32.state_dict().items()})
    gen = torch.Generator(device="cpu").manual_seed(98)
    ids = torch.randint(0, cfg.vocab_size, (B, sum(CHUNKS) + DECODE), generator=gen).to(cuda)

    want = _run(ref32, DynamicCache(config=cfg), ids)
    # the sinks matter at this bar: without them the fp32 logits move far more than it allows
    sinks = [layer.self_attn.sinks.clone() for layer in ref32.model.layers]
    for layer in ref32.model.layers:
        layer.self_attn.sinks.fill_(-1e4)
    no_sink = _run(ref32, DynamicCache(config=cfg), ids)
    for layer, sk in zip(ref32.model.layers, sinks):
        layer.self_attn.sinks.copy_(sk)
    model.set_attn_implementation("eager")
    eager16 = _run(model, DynamicCache(config=cfg), ids)
    for i in range(1, len(want)):
        bar = 1.5 * (eager16[i] - want[i]).abs().max().item() + 0.005
        assert (no_sink[i] - want[i]).abs().max().item() > 3 * bar, f"step {i}: sinks too weak to test"
    pool = KVPool(num_layers=cfg.num_hidden_layers, num_blocks=64, block_size=16, num_kv_heads=2, head_dim=64,
                  device=cuda)
    cache = PagedCache(pool, [20, 21, 22])
    model.set_attn_implementation(register())
    got = _run(model, cache, ids)
    print("step  |paged-fp32|  |eager16-fp32|")
    for i, (g, e, w) in enumerate(zip(got, eager16, want)):
        assert torch.isfinite(g).all(), f"step {i}: non-finite logits"
        d_paged = (g - w).abs().max().item()
        d_eager = (e - w).abs().max().item()
        print(f"{i:4d}  {d_paged:.4f}  {d_eager:.4f}")
        assert d_paged <= 1.5 * d_eager + 0.005, f"step {i}: paged {d_paged:.4f} vs eager bf16 {d_eager:.4f}"

