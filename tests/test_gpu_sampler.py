"""GPU parity of the token sampler against the numpy oracle (same float32 steps,
same counter-based random stream): tokens and sampling masks equal, processed
logprobs within 1e-4; a one-launch draw of 8,192 rows matches the kept
softmax it samples from."""

import numpy as np
import pytest
import torch

from oracle import paged
from oracle import sampler as S
from wavelet_amd import sample, synth
from wavelet_amd.sampler import seen_bitmap

pytestmark = pytest.mark.gpu

# per-row (temperature, top_k, top_p, min_p, repetition_penalty)
ROWS = [(1.0, 0, 1.0, 0.0, 1.0), (0.7, 50, 1.0, 0.0, 1.0), (1.0, 0, 0.9, 0.0, 1.0), (1.2, 0, 1.0, 0.05, 1.0),
        (0.8, 40, 0.8, 0.01, 1.3), (0.0, 0, 1.0, 0.0, 1.0), (1.0, 1, 1.0, 0.0, 1.0), (0.6, 0, 0.3, 0.0, 1.1)]


def _check_rows(cuda, x, rows, seen_lists, seeds, step, dtype):
    """Run `sample` on float32 logits x [B, V] (as dtype) and compare every row with the oracle."""
    B, vocab = x.shape
    if dtype == torch.bfloat16:
        bits = paged.f32_to_bf16(x)
        x = paged.bf16_to_f32(bits)
        logits = torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(x).to(cuda)
    seen = seen_bitmap(seen_lists, vocab)
    T, K, P, MP, RP = (np.array([r[i] for r in rows]) for i in range(5))
    tokens, logprobs, mask, counts = sample(
        logits, temperature=torch.tensor(T, dtype=torch.float32, device=cuda),
        top_k=torch.tensor(K, dtype=torch.int32, device=cuda), top_p=torch.tensor(P, dtype=torch.float32, device=cuda),
        min_p=torch.tensor(MP, dtype=torch.float32, device=cuda),
        repetition_penalty=torch.tensor(RP, dtype=torch.float32, device=cuda),
        seen=torch.from_numpy(seen).to(cuda), seeds=torch.from_numpy(seeds).to(cuda), step=step, return_mask=True)
    tokens, logprobs = tokens.cpu().numpy(), logprobs.cpu().numpy()
    mask, counts = mask.cpu().numpy().view(np.uint32), counts.cpu().numpy()
    bits = ((mask[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(B, -1)[:, :vocab].astype(bool)
    for r in range(B):
        seen_row = np.zeros(vocab, bool)
        seen_row[seen_lists[r]] = True
        tok, lp, kept, amb = S.sample_row(x[r], temperature=T[r], top_k=int(K[r]), top_p=P[r], min_p=MP[r],
                                          repetition_penalty=RP[r], seen=seen_row, seed=int(seeds[r]), step=step)
        assert counts[r] == bits[r].sum(), f"row {r}: count"
        if not amb:
            np.testing.assert_array_equal(bits[r], kept, err_msg=f"row {r} ({rows[r]}): kept set")
        if tokens[r] != tok:  # only a float32 near-tie of the race may differ
            xr = x[r].copy()
            if RP[r] != 1.0:
                xr = np.where(seen_row, np.where(xr > 0, xr / np.float32(RP[r]), xr * np.float32(RP[r])), xr)
            xr = xr * (np.float32(1.0) / np.float32(T[r]) if T[r] >= 1e-5 else np.float32(1.0))
            le = S.log_exp_variates(int(seeds[r]), step, vocab)
            s_gpu, s_ref = xr[tokens[r]] - le[tokens[r]], xr[tok] - le[tok]
            assert abs(float(s_gpu) - float(s_ref)) < 1e-4 and bits[r][tokens[r]], f"row {r}: token {tokens[r]} vs {tok}"
        else:
            assert abs(logprobs[r] - lp) < 1e-4, f"row {r}: logprob {logprobs[r]} vs {lp}"


@pytest.mark.parametrize("vocab", [151936, 32001, 1000])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sampler_matches_oracle(cuda, vocab, dtype):
    B = len(ROWS)
    x = (synth.normal(synth.stream_key("smp", vocab, str(dtype)), B * vocab) * 4.0).astype(np.float32).reshape(B, vocab)
    rng = np.random.default_rng(vocab)
    seen_lists = [rng.integers(0, vocab, 64) for _ in range(B)]
    seeds = np.arange(B, dtype=np.int64) * 1000 + 17
    _check_rows(cuda, x, ROWS, seen_lists, seeds, 5, dtype)


def test_sampler_list_and_full_row_paths(cuda):
    """Rows that take the one-histogram path (threshold near the max, at most 4,096 candidates) and rows
    that take the full-row radix passes: a list that would overflow (top_k 5,000; flat logits under
    top_p), a threshold in the open bin (the 2nd largest 100 below the max)."""
    V = 151936
    rows = [(1.0, 3000, 1.0, 0.0, 1.0), (1.0, 5000, 1.0, 0.0, 1.0), (1.0, 2, 1.0, 0.0, 1.0),
            (1.0, 0, 0.5, 0.0, 1.0), (0.5, 20, 0.7, 0.0, 1.0), (1.0, 0, 0.999, 0.0, 1.0)]
    x = (synth.normal(synth.stream_key("smp-paths"), len(rows) * V) * 4.0).astype(np.float32).reshape(len(rows), V)
    x[2] = -200.0
    x[2, 7] = 0.0
    x[2, 99] = -100.0
    x[2, 1234] = -100.0  # a tie at the threshold: both kept
    x[3] = 0.0  # flat: every token in bin 0
    seen_lists = [np.zeros(0, np.int64) for _ in rows]
    seeds = np.arange(len(rows), dtype=np.int64) + 3
    _check_rows(cuda, x, rows, seen_lists, seeds, 2, torch.float32)


def test_sampler_capture_paths(cuda):
    """Rows for the one-capture-pass list: top_k whose range holds fewer kept tokens than k (min_p),
    k equal to the thread count, a flat row whose range overflows the list (histogram, then full-row
    passes), top_p alone and top_k + top_p on peaked logits (the list holds the threshold), greedy
    with top_k (the list's argmax)."""
    V = 151936
    rows = [(1.0, 50, 1.0, 0.5, 1.0), (1.0, 1024, 1.0, 0.0, 1.0), (1.0, 20, 1.0, 0.0, 1.0),
            (1.0, 0, 0.9, 0.0, 1.0), (0.7, 50, 0.9, 0.0, 1.0), (0.0, 50, 1.0, 0.0, 1.0), (1.0, 0, 0.995, 0.0, 1.2)]
    x = (synth.normal(synth.stream_key("smp-capture"), len(rows) * V) * 4.0).astype(np.float32).reshape(len(rows), V)
    x[2] = 0.0
    x[3:] *= 10.0
    rng = np.random.default_rng(7)
    seen_lists = [rng.integers(0, V, 200) for _ in rows]
    seeds = np.arange(len(rows), dtype=np.int64) + 11
    _check_rows(cuda, x, rows, seen_lists, seeds, 4, torch.float32)


def test_sampler_vocab_beyond_lds_mask(cuda):
    """300,000 tokens (9,375 mask words): the list path keeps the full-row final pass."""
    V = 300000
    rows = [(0.7, 50, 0.9, 0.0, 1.0), (1.0, 0, 0.9, 0.0, 1.0), (1.0, 0, 1.0, 0.0, 1.0)]
    x = (synth.normal(synth.stream_key("smp-300k"), len(rows) * V) * 40.0).astype(np.float32).reshape(len(rows), V)
    seen_lists = [np.zeros(0, np.int64) for _ in rows]
    seeds = np.arange(len(rows), dtype=np.int64) + 5
    _check_rows(cuda, x, rows, seen_lists, seeds, 1, torch.bfloat16)


def test_sampler_draws_match_kept_softmax(cuda):
    """8,192 independent rows (seeds 0..8191) of the same 8 logits in one launch."""
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 3.0, -5.0, 1.5], np.float32)
    n = 8192
    logits = torch.from_numpy(np.tile(x, (n, 1))).to(cuda)
    tok, _, mask, _ = sample(logits, top_k=5, seeds=torch.arange(n, dtype=torch.int64, device=cuda), step=11,
                             return_mask=True)
    counts = np.bincount(tok.cpu().numpy(), minlength=8)
    kept = np.zeros(8, bool)
    kept[np.argsort(x)[-5:]] = True
    p = np.where(kept, np.exp(x - x.max()), 0.0)
    p /= p.sum()
    assert np.all(counts[~kept] == 0)
    np.testing.assert_allclose(counts / n, p, atol=5 * np.sqrt(0.25 / n))
    assert np.all(mask.cpu().numpy()[:, 0] == mask.cpu().numpy()[0, 0])


def test_sampler_edge_rows(cuda):
    """A row with one finite logit, greedy ties (lowest index), top_k beyond the support."""
    V = 300
    x = np.full((3, V), -np.inf, np.float32)
    x[0, 123] = 0.5
    x[1, :] = 1.0
    x[1, [7, 200]] = 2.0
    x[2, :10] = np.linspace(0, 1, 10)
    tok, lp, mask, counts = sample(torch.from_numpy(x).to(cuda), temperature=torch.tensor([1.0, 0.0, 1.0], device=cuda),
                                   top_k=torch.tensor([5, 0, 50], dtype=torch.int32, device=cuda), return_mask=True)
    tok, lp, counts = tok.cpu().numpy(), lp.cpu().numpy(), counts.cpu().numpy()
    assert tok[0] == 123 and abs(lp[0]) < 1e-6 and counts[0] == 1
    assert tok[1] == 7 and counts[1] == V
    assert counts[2] == 10 and tok[2] < 10


def test_sampler_out_buffers(cuda):
    """Preallocated outputs give the same results; wrong shapes or dtypes are rejected."""
    B, V = 4, 5000
    x = torch.from_numpy((synth.normal(synth.stream_key("smp-out"), B * V) * 3.0).astype(np.float32).reshape(B, V)).to(cuda)
    seeds = torch.arange(B, dtype=torch.int64, device=cuda)
    ref = sample(x, temperature=0.8, top_k=20, seeds=seeds, step=3, return_mask=True)
    words = (V + 31) // 32
    out = (torch.empty(B, dtype=torch.int64, device=cuda), torch.empty(B, dtype=torch.float32, device=cuda),
           torch.empty((B, words), dtype=torch.int32, device=cuda), torch.empty(B, dtype=torch.int32, device=cuda))
    got = sample(x, temperature=0.8, top_k=20, seeds=seeds, step=3, return_mask=True, out=out)
    for r, g, o in zip(ref, got, out):
        assert g is o and torch.equal(r, g)
    with pytest.raises(ValueError, match="mask"):
        sample(x, return_mask=True, out=(out[0], out[1], None, out[3]))
    with pytest.raises(ValueError, match="logprobs"):
        sample(x, out=(out[0], out[1].double(), None, None))


def test_sampler_parameter_ranges(cuda):
    """Scalars outside the sampling config's ranges are rejected; a per-row min_p above 1 (not read
    back) keeps the row's maximum, as min_p = 1 does."""
    V = 2000
    x = (synth.normal(synth.stream_key("smp-ranges"), 2 * V) * 3.0).astype(np.float32).reshape(2, V)
    logits = torch.from_numpy(x).to(cuda)
    for kw in (dict(min_p=1.5), dict(min_p=-0.1), dict(top_p=0.0), dict(top_p=1.2), dict(temperature=-1.0),
               dict(repetition_penalty=0.0)):
        with pytest.raises(ValueError):
            sample(logits, **kw)
    rows = [(1.0, 0, 1.0, 2.0, 1.0), (0.7, 5, 1.0, 1.0, 1.0)]
    _check_rows(cuda, x, rows, [np.zeros(0, np.int64)] * 2, np.arange(2, dtype=np.int64), 1, torch.float32)
    tok = sample(logits, min_p=torch.tensor([2.0, 2.0], device=cuda))[0].cpu().numpy()
    np.testing.assert_array_equal(tok, np.argmax(x, axis=1))
