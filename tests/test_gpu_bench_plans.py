"""Parity at the launch plans the benchmark times, at the workloads' full sizes.

Every plan here is built by the benchmark's own constructor calls
(``bench.gqa_cache`` -- the caches and their read policy -- then
``bench.gqa_plan`` / ``bench.mla_plan``: fused append + attention, the
library's partition, dispatch order and waves per workgroup) on two layers of
the full-size workload, so the kernel instantiations and launch shapes under
test are the ones the bench line reports -- e.g. the headline's
``decode_gqa_kernel<128,false,true,8,1>`` (streamed reads) with 512-token
partitions and one workgroup per (sequence, KV head), no merge, and the fp8
groups' kernels: the group-aware one (prompt blocks cached, the members' own
tokens streamed, the group order) and the plain one (everything cached).

Per layer, after one ``run()``:

* the cache equals its pre-step copy with every sequence's new token written
  (bf16: by torch indexing; fp8: by the oracle's ``append_fp8`` on the touched
  blocks) -- bit for bit, over the whole cache;
* every output is finite, and at least 8 sequences (all query heads, including
  the longest and the shortest context) match the float64 oracle to the
  attention bar of ``kvcase.check_attention`` (max |err| <= 2e-2 outright);
* NaN fills every slot no context owns and the new tokens' slots before the
  step, and guard pads of NaN surround each cache, output and workspace tensor
  and must be intact after it.

The error of the reference's bf16 path (the oracle with P cast to bf16 before
PV, as ``_eager_sparse_attention`` does at
wavelet/trainer/models/deepseek_v4/attention.py:94-96, output rounded to
bf16) against the same float64 oracle is printed beside the kernel's (and
appended as JSON to ``$WKV_PARITY_LOG`` when that is set).
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

import bench
from kvcase import Guarded, assert_guards, bits_of, check_attention, guard_cache, guarded_workspace
from oracle import fp8, paged
from wavelet_amd import MLALatentCache, _lib, decode_plan, synth

pytestmark = pytest.mark.gpu

LAYERS = 2
BF16_NAN = 0x7FC0
FP8_NAN = 0x7F


def _log(rec: dict) -> None:
    print(json.dumps(rec))
    path = os.environ.get("WKV_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")


def _owned(w) -> np.ndarray:
    """[NB, BS] True where some context covers the slot before this step (the new tokens excluded)."""
    own = np.zeros((w.num_blocks, w.block_size), bool)
    for i in range(w.batch):
        pos = np.arange(int(w.context_lens[i]) - 1)
        own[w.block_tables[i][pos // w.block_size], pos % w.block_size] = True
    return own


def _checked_sequences(w, n: int = 8) -> np.ndarray:
    L = w.context_lens
    pick = {int(np.argmax(L)), int(np.argmin(L))}
    for i in np.linspace(0, w.batch - 1, n).astype(int):
        if len(pick) >= n:
            break
        pick.add(int(i))
    return np.array(sorted(pick))


def _compact(w, seqs):
    """Blocks the chosen sequences read, as a compact pool: (block ids, compact tables, lengths)."""
    L = w.context_lens[seqs].astype(np.int64)
    nb = (L + w.block_size - 1) // w.block_size
    ids = np.unique(np.concatenate([w.block_tables[i, :n] for i, n in zip(seqs, nb)]))
    bt = np.full((len(seqs), int(nb.max())), -1, np.int32)
    for j, (i, n) in enumerate(zip(seqs, nb)):
        bt[j, :n] = np.searchsorted(ids, w.block_tables[i, :n])
    return ids, bt, L.astype(np.int32)


def _gqa_buffers(cuda, w, kv_dtype: str, std: float):
    """Guarded per-layer caches (random owned slots, NaN elsewhere), step inputs and guarded outputs."""
    gen = torch.Generator(device=cuda)
    gen.manual_seed(20261202)
    B, HQ, HKV, D, BS = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.block_size
    own = torch.from_numpy(_owned(w)).to(cuda)
    caches, guards, qs, ks, vs, outs = [], [], [], [], [], []
    for _ in range(LAYERS):
        c = bench.gqa_cache(w, kv_dtype, cuda)  # the bench's own caches (and read policy)
        assert c.shared_blocks == (w.group_size > 1)
        if kv_dtype == "bf16":
            c.k.normal_(generator=gen).mul_(std)
            c.v.normal_(generator=gen).mul_(std)
            c.k.view(torch.int16).masked_fill_(~own[:, None, None, :, None], BF16_NAN)
            c.v.view(torch.int16).masked_fill_(~own[:, None, None, :], BF16_NAN)
        else:  # finite e4m3 codes in owned slots (no 0x7F / 0xFF), 2^-8 scales, NaN codes elsewhere
            for t in (c.k, c.v):
                t.copy_(torch.randint(0, 256, t.shape, generator=gen, device=cuda, dtype=torch.int32)
                        .to(torch.uint8) & 0xF7)
            c.k.masked_fill_(~own[:, None, None, :, None], FP8_NAN)
            c.v.masked_fill_(~own[:, None, None, :], FP8_NAN)
            c.k_scale.fill_(2.0 ** -8)
            c.v_scale.fill_(2.0 ** -8)
        guards += guard_cache(c)
        caches.append(c)
        qs.append((torch.randn((B, HQ, D), generator=gen, device=cuda) * std).to(torch.bfloat16))
        ks.append((torch.randn((B, HKV, D), generator=gen, device=cuda) * std).to(torch.bfloat16))
        vs.append((torch.randn((B, HKV, D), generator=gen, device=cuda) * std).to(torch.bfloat16))
        g = Guarded((B, HQ, D), torch.bfloat16, cuda)
        guards.append(g)
        outs.append(g.t)
    return caches, guards, qs, ks, vs, outs


def _expected_bf16_cache(c, key, value, slots, BS):
    """The pre-step cache with each sequence's new token written, by torch indexing."""
    k, v = c.k.clone(), c.v.clone()
    blk, off = slots // BS, slots % BS
    B, H, D = key.shape
    k[blk, :, :, off, :] = key.view(B, H, D // 8, 8)
    v[blk, :, :, off] = value
    return k, v


def _expected_fp8_cache(c, key, value, slots, BS):
    """The pre-step cache with the new tokens appended by the oracle's fp8 rule (touched blocks only)."""
    k, v, ksc, vsc = c.k.clone(), c.v.clone(), c.k_scale.clone(), c.v_scale.clone()
    blocks = torch.unique(slots // BS)
    kb, vb = bits_of(k[blocks]), bits_of(v[blocks])
    ks_, vs_ = ksc[blocks].cpu().numpy(), vsc[blocks].cpu().numpy()
    s_np = slots.cpu().numpy()
    local = np.searchsorted(blocks.cpu().numpy(), s_np // BS) * BS + s_np % BS
    paged.append_fp8(kb, vb, ks_, vs_, bits_of(key), bits_of(value), local)
    k[blocks] = torch.from_numpy(kb).to(k.device)
    v[blocks] = torch.from_numpy(vb).to(v.device)
    ksc[blocks] = torch.from_numpy(ks_).to(k.device)
    vsc[blocks] = torch.from_numpy(vs_).to(k.device)
    return k, v, ksc, vsc


def _oracle_gqa(c, w, q, seqs):
    ids, bt, lens = _compact(w, seqs)
    idx = torch.from_numpy(ids).to(c.k.device)
    kp, vp = bits_of(c.k[idx]), bits_of(c.v[idx])
    qf = paged.bf16_to_f32(bits_of(q[torch.from_numpy(seqs).to(q.device)]))
    n, BS, H, D = len(ids), w.block_size, w.num_kv_heads, w.head_dim
    if c.kv_dtype == "fp8_e4m3":
        ks, vs = c.k_scale[idx].cpu().numpy(), c.v_scale[idx].cpu().numpy()
        kf = fp8.dequantize(paged.k_logical(kp).reshape(n, BS, H, D), ks[:, None, :, None])
        vf = fp8.dequantize(paged.v_logical(vp), vs[:, None, :, None])
    else:
        kl, vl = paged.logical_kv(kp, vp)
        kf, vf = paged.bf16_to_f32(kl), paged.bf16_to_f32(vl)
    ref = paged.decode_gqa(qf, kf, vf, bt, lens, w.scale)
    ref_bf16 = paged.decode_gqa(qf, kf, vf, bt, lens, w.scale, p_bf16=True)
    ref_bf16 = paged.bf16_to_f32(paged.f32_to_bf16(ref_bf16.astype(np.float32)))
    return ref, ref_bf16


def _run_gqa_plan(cuda, name, w, kv_dtype, std=1.0, grouped=False, expect_plan=None):
    torch.cuda.synchronize()
    print(f"case {name}: B={w.batch} {w.num_q_heads}/{w.num_kv_heads} d={w.head_dim} {kv_dtype} "
          f"L=[{int(w.context_lens.min())}, {int(w.context_lens.max())}] grouped={grouped}", flush=True)
    lib = _lib.load()
    max_seq = int(w.context_lens.max())
    if grouped:
        need = lib.wkv_grouped_decode_workspace_size(w.batch, w.num_q_heads, w.head_dim, max_seq, w.prefix_len, 0)
    else:
        need = lib.wkv_decode_workspace_size(w.batch, w.num_q_heads, w.head_dim, max_seq, 0)
    ws = guarded_workspace(cuda, int(need))
    caches, guards, qs, ks, vs, outs = _gqa_buffers(cuda, w, kv_dtype, std)
    guards.append(ws)
    step = bench.gqa_plan(torch, cuda, w, caches, qs, ks, vs, outs, 0, grouped)
    plan = decode_plan(w.batch, w.num_kv_heads, max_seq, w.block_size, 0)
    print(f"  plan: partition {plan[0]}, {plan[1]} waves/workgroup, {plan[2]} chunks; ordered={step.ordered}")
    if expect_plan is not None:
        assert plan == expect_plan, f"{name}: the bench's plan is {plan}, expected {expect_plan}"
    slots = step.slot_mapping
    BS = w.block_size
    if kv_dtype == "bf16":
        expect = [_expected_bf16_cache(c, k, v, slots, BS) for c, k, v in zip(caches, ks, vs)]
    else:
        expect = [_expected_fp8_cache(c, k, v, slots, BS) for c, k, v in zip(caches, ks, vs)]
    step.run()
    assert_guards(guards, name)
    seqs = _checked_sequences(w)
    for layer, c in enumerate(caches):
        if kv_dtype == "bf16":
            ek, ev = expect[layer]
            assert torch.equal(c.k.view(torch.int16), ek.view(torch.int16)), f"{name} layer {layer}: K cache"
            assert torch.equal(c.v.view(torch.int16), ev.view(torch.int16)), f"{name} layer {layer}: V cache"
        else:
            ek, ev, eks, evs = expect[layer]
            assert torch.equal(c.k, ek) and torch.equal(c.v, ev), f"{name} layer {layer}: fp8 K/V cache"
            assert torch.equal(c.k_scale, eks) and torch.equal(c.v_scale, evs), f"{name} layer {layer}: scales"
        out = outs[layer]
        assert bool(torch.isfinite(out.float()).all()), f"{name} layer {layer}: non-finite output"
        ref, ref_bf16 = _oracle_gqa(c, w, qs[layer], seqs)
        got = paged.bf16_to_f32(bits_of(out[torch.from_numpy(seqs).to(cuda)]))
        a, r = check_attention(got, ref, f"{name} layer {layer}")
        ra, rr = paged.max_abs_and_rel(ref_bf16, ref)
        _log({"case": name, "layer": layer, "plan": list(plan), "sequences": seqs.tolist(), "gpu_max_abs": a,
              "gpu_rel_l2": r, "reference_bf16_max_abs": ra, "reference_bf16_rel_l2": rr})


def test_headline_plan_qwen3_4b_b64_l4096(cuda):
    """The bench's default line: 36 layers of this in the timed step."""
    w = synth.qwen3_4b_workload(batch=64, context=4096)
    _run_gqa_plan(cuda, "qwen3-4b", w, "bf16", expect_plan=(512, 8, 1))


def test_plan_qwen3_4b_variable_lengths_b64(cuda):
    w = synth.qwen3_4b_workload(batch=64, context=None)
    _run_gqa_plan(cuda, "qwen3-4b-var", w, "bf16")


def test_plan_qwen25_05b_b128(cuda):
    w = synth.qwen25_05b_workload()
    _run_gqa_plan(cuda, "qwen2.5-0.5b", w, "bf16", std=1 / 8)


@pytest.mark.parametrize("grouped", [False, True])
def test_plan_qwen25_7b_fp8_groups_256_sequences(cuda, grouped):
    """All 32 groups x 8 members; the group-aware plan is the bench default, the plain one
    is --plain-decode."""
    w = synth.qwen25_7b_group_workload()
    _run_gqa_plan(cuda, "qwen2.5-7b-groups" + ("-grouped" if grouped else ""), w, "fp8_e4m3", grouped=grouped)


def test_plan_deepseek_v3_mla_b32(cuda):
    """128 heads over the 576-wide latent, B=32, L=4096, block 64, fused latent append."""
    w = synth.deepseek_v3_mla_workload()
    torch.cuda.synchronize()
    print(f"case deepseek-v3-mla: B={w.batch} L={int(w.context_lens.max())}", flush=True)
    R, P, H, B, BS = 512, 64, 128, w.batch, w.block_size
    lib = _lib.load()
    need = lib.wkv_mla_workspace_size(B, H, R, int(w.context_lens.max()), 0)
    ws = guarded_workspace(cuda, int(need))
    gen = torch.Generator(device=cuda)
    gen.manual_seed(20261202)
    own = torch.from_numpy(_owned(w)).to(cuda)
    caches, guards, qn, qp, kc, kp, outs = [], [ws], [], [], [], [], []
    for _ in range(LAYERS):
        c = MLALatentCache(w.num_blocks, BS, R, P, device=cuda)
        c.latent.normal_(generator=gen)
        c.latent.view(torch.int16).masked_fill_(~own[:, :, None], BF16_NAN)
        guards += guard_cache(c)
        caches.append(c)
        qn.append(torch.randn((B, H, R), generator=gen, device=cuda).to(torch.bfloat16))
        qp.append(torch.randn((B, H, P), generator=gen, device=cuda).to(torch.bfloat16))
        kc.append(torch.randn((B, R), generator=gen, device=cuda).to(torch.bfloat16))
        kp.append(torch.randn((B, P), generator=gen, device=cuda).to(torch.bfloat16))
        g = Guarded((B, H, R), torch.bfloat16, cuda)
        guards.append(g)
        outs.append(g.t)
    step = bench.mla_plan(torch, cuda, w, caches, qn, qp, kc, kp, outs, 0)
    slots = torch.from_numpy(w.new_token_slots()).to(cuda)
    expect = []
    for c, a, b in zip(caches, kc, kp):
        lat = c.latent.clone().view(-1, R + P)
        lat[slots] = torch.cat([a, b], dim=1)
        expect.append(lat)
    step.run()
    assert_guards(guards, "deepseek-v3-mla")
    seqs = _checked_sequences(w)
    ids, bt, lens = _compact(w, seqs)
    idx = torch.from_numpy(ids).to(cuda)
    sel = torch.from_numpy(seqs).to(cuda)
    for layer, c in enumerate(caches):
        assert torch.equal(c.latent.view(-1, R + P).view(torch.int16), expect[layer].view(torch.int16)), \
            f"mla layer {layer}: latent cache"
        out = outs[layer]
        assert bool(torch.isfinite(out.float()).all()), f"mla layer {layer}: non-finite output"
        lat = paged.bf16_to_f32(bits_of(c.latent[idx]))
        q = paged.bf16_to_f32(bits_of(torch.cat([qn[layer], qp[layer]], dim=2)[sel]))
        ref = paged.decode_mla(q, lat, bt, lens, w.scale)
        ref_bf16 = paged.decode_mla(q, lat, bt, lens, w.scale, p_bf16=True)
        ref_bf16 = paged.bf16_to_f32(paged.f32_to_bf16(ref_bf16.astype(np.float32)))
        got = paged.bf16_to_f32(bits_of(out[sel]))
        a, r = check_attention(got, ref, f"mla layer {layer}")
        ra, rr = paged.max_abs_and_rel(ref_bf16, ref)
        _log({"case": "deepseek-v3-mla", "layer": layer, "sequences": seqs.tolist(), "gpu_max_abs": a,
              "gpu_rel_l2": r, "reference_bf16_max_abs": ra, "reference_bf16_rel_l2": rr})

