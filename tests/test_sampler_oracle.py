"""Pins of the sampler oracle (CPU): kept sets against straightforward torch
formulations of min_p / top_k / top_p, the exponential race against the
softmax it must draw from, greedy rows, penalties and logprobs."""

import math

import numpy as np
import pytest
import torch

from oracle import sampler as S
from wavelet_amd import synth


def _logits(name, v, scale=3.0):
    return (synth.normal(synth.stream_key("sampler", name), v) * scale).astype(np.float32)


def _torch_kept(x, top_k=0, top_p=1.0, min_p=0.0):
    x = torch.from_numpy(x.astype(np.float64))
    keep = torch.ones_like(x, dtype=torch.bool)
    if min_p > 0:
        p = torch.softmax(x, 0)
        keep &= p >= min_p * p.max()
    if 0 < top_k < x.numel():
        kth = torch.topk(torch.where(keep, x, torch.tensor(-math.inf, dtype=x.dtype)), top_k).values[-1]
        keep &= x >= kth
    if top_p < 1.0:
        p = torch.softmax(torch.where(keep, x, torch.tensor(-math.inf, dtype=x.dtype)), 0)
        sp, order = torch.sort(p, descending=True)
        above = torch.cumsum(sp, 0) - sp  # mass strictly before in sorted order (no ties here)
        k = torch.zeros_like(keep)
        k[order] = above < top_p
        keep &= k
    return keep.numpy()


def test_kept_sets_match_torch_formulations():
    for i, (tk, tp, mp) in enumerate([(0, 1.0, 0.0), (50, 1.0, 0.0), (0, 0.9, 0.0), (0, 1.0, 0.05), (40, 0.8, 0.01),
                                      (1, 1.0, 0.0), (0, 0.3, 0.0)]):
        x = _logits(f"k{i}", 5000)
        _, _, kept, amb = S.sample_row(x, top_k=tk, top_p=tp, min_p=mp)
        assert not amb
        np.testing.assert_array_equal(kept, _torch_kept(x, tk, tp, mp), err_msg=f"k={tk} p={tp} min_p={mp}")


def test_exponential_race_draws_from_the_kept_softmax():
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 3.0, -5.0, 1.5], np.float32)
    n = 20000
    counts = np.zeros(x.size)
    for step in range(n):
        tok, _, kept, _ = S.sample_row(x, top_k=5, seed=7, step=step)
        counts[tok] += 1
    p = np.where(kept, np.exp(x - x.max()), 0.0)
    p /= p.sum()
    assert np.all(counts[~kept] == 0)
    # multinomial standard error sqrt(p(1-p)/n) <= 0.0036: allow 5 sigma
    np.testing.assert_allclose(counts / n, p, atol=0.018)


def test_greedy_logprob_and_penalty():
    x = _logits("g", 1000)
    tok, lp, kept, _ = S.sample_row(x, temperature=0.0)
    assert tok == int(np.argmax(x)) and kept.all()
    ref = float(x[tok] - np.log(np.exp(x.astype(np.float64) - x.max()).sum()) - x.max())
    assert abs(lp - ref) < 1e-5
    # logprob of a sampled token = log-softmax over the kept set of x / T
    tok, lp, kept, _ = S.sample_row(x, temperature=0.7, top_k=20, seed=3, step=1)
    xt = (x * np.float32(1 / np.float32(0.7))).astype(np.float64)
    ref = xt[tok] - np.log(np.exp(xt[kept]).sum())
    assert kept.sum() == 20 and abs(lp - ref) < 1e-5
    # repetition penalty divides positive and multiplies negative seen logits
    seen = np.zeros(1000, bool)
    seen[[int(np.argmax(x)), int(np.argmin(x))]] = True
    tok2, _, _, _ = S.sample_row(x, temperature=0.0, repetition_penalty=1e6, seen=seen)
    assert tok2 != int(np.argmax(x)) and tok2 == int(np.argsort(x)[-2])


def test_hash_stream_is_fixed():
    """The random stream is part of the contract (GPU and oracle draw the same
    variates): pin its first values."""
    v = S.log_exp_variates(seed=1, step=0, n=4)
    u = np.exp(-np.exp(v))
    assert np.all((u > 0) & (u < 1))
    # the published splitmix64 sequence from state 0: mix(gamma), mix(2 gamma)
    h = S.mix64(np.array([0x9E3779B97F4A7C15, 0x3C6EF372FE94F82A], np.uint64))
    assert [int(x) for x in h] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]


def test_uniform_stays_inside_the_open_interval():
    """u from the extreme hash values stays strictly inside (0, 1) in float32, so
    every race score is finite (the top 24-bit value would round to u = 1)."""
    for top in (np.uint64(0), np.uint64(0xFFFFFFFFFFFFFFFF)):
        u = ((top >> np.uint64(41)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 8388608.0)
        assert 0.0 < float(u) < 1.0 and np.isfinite(np.log(-np.log(u)))
    u24 = ((np.uint64(0xFFFFFFFFFFFFFFFF) >> np.uint64(40)).astype(np.float32) + np.float32(0.5)) * np.float32(
        1.0 / 16777216.0)
    assert float(u24) == 1.0  # the mapping this replaced
    v = S.log_exp_variates(seed=123, step=7, n=200_000)
    assert np.all(np.isfinite(v))


def test_min_p_above_one_keeps_the_maximum():
    x = np.array([0.5, 2.0, -1.0, 2.0, 1.9], np.float32)
    tok, lp, kept, _ = S.sample_row(x, min_p=3.0, seed=1, step=0)
    np.testing.assert_array_equal(kept, [False, True, False, True, False])  # the tied maxima
    assert tok in (1, 3) and abs(lp - np.log(0.5)) < 1e-6


@pytest.mark.parametrize("kw", [dict(min_p=1.5), dict(min_p=-0.1), dict(top_p=0.0), dict(top_p=1.2),
                                dict(temperature=-1.0), dict(repetition_penalty=0.0)])
def test_sample_rejects_out_of_range_scalars(kw):
    """Checked on the host before anything touches a device (the reference config's ranges)."""
    from wavelet_amd import sample
    with pytest.raises(ValueError, match=next(iter(kw))):
        sample(torch.zeros((2, 10)), **kw)
