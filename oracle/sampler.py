"""The token sampler restated in numpy (oracle; tests and the CPU baseline only).

The semantics the HIP sampler implements (wkv_sample), step by step in float32
as the kernel computes them: repetition penalty on seen tokens, temperature
(greedy below 1e-5), min_p, top_k (ties kept), top_p (token i kept iff the
fixed-point softmax mass of strictly larger tokens is below top_p of the kept
mass), then the exponential race with the counter-based hash. vLLM's sampler
(the reference's generation path, wavelet/inference/engine.py:69-90, :795-805,
logprobs_mode="processed_logprobs") is absent here; its order of operations
(penalties, temperature, min_p, top-k/top-p, exponential race) is followed,
its tie-breaking and summation order are not pinned (parity unpinned against
vLLM itself; pinned here against straightforward torch formulations).
"""

from __future__ import annotations

import numpy as np

GREEDY_EPS = np.float32(1e-5)
GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def mix64(z: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser on uint64 arrays (wrapping arithmetic)."""
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def order_key(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 keys of float32 values; NaN -> 0."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    k = np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    return np.where(np.isnan(x), np.uint32(0), k)


def log_exp_variates(seed: int, step: int, n: int) -> np.ndarray:
    """ln(E_i) of the Exp(1) variates E_i = -ln(u_i), i = 0..n-1 (float32)."""
    with np.errstate(over="ignore"):
        stream = mix64(np.uint64(seed) + np.uint64(step) * GOLDEN)
        h = mix64(stream + np.arange(n, dtype=np.uint64))
    # 23 hash bits: u in [2^-24, 1 - 2^-24], exact in float32 (with 24 bits the
    # top value rounds to 1.0, giving E = 0 and an infinite race score)
    u = ((h >> np.uint64(41)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 8388608.0)
    # (the kernel takes both logarithms as the hardware log2 times ln 2: within an
    # ulp or two of these, so race scores agree to ~1e-6 and only near-ties of
    # the race may pick another token)
    return np.log(-np.log(u)).astype(np.float32)


def _radix_key_topk(keys: np.ndarray, k: int) -> np.uint32 | None:
    """Key of the k-th largest (ties counted), or None if fewer than k."""
    if keys.size < k:
        return None
    return np.sort(keys)[::-1][k - 1]


def sample_row(logits, *, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0, seen=None,
               seed=0, step=0):
    """One row -> (token, processed logprob, kept bool mask, ambiguous).

    ``ambiguous`` flags a top-p boundary within 1e-6 of the target mass, where
    a one-ulp difference in exp could move the threshold.
    """
    l = np.asarray(logits, dtype=np.float32).copy()
    pen = np.float32(repetition_penalty)
    if seen is not None and pen != np.float32(1.0):
        s = np.asarray(seen, dtype=bool)
        l = np.where(s, np.where(l > 0, l / pen, l * pen), l).astype(np.float32)
    t = np.float32(temperature)
    greedy = t < GREEDY_EPS
    inv_t = np.float32(1.0) if greedy else np.float32(1.0) / t
    x = (l * inv_t).astype(np.float32)
    finite = np.isfinite(x)
    if not finite.any():
        return 0, -np.inf, np.zeros(x.shape, bool), False
    mx = np.float32(x[finite].max())
    keys = order_key(x)
    key_lo = order_key(np.float32(-3.402823466e38))
    if min_p > 0:  # (capped at the maximum's key: min_p above 1 still keeps the maximum)
        key_lo = max(key_lo, min(order_key(np.float32(mx + np.float32(np.log(np.float32(min_p))))), order_key(mx)))
    v = x.size
    if 0 < top_k < v:
        kk = _radix_key_topk(keys[keys >= key_lo], int(top_k))
        if kk is not None:
            key_lo = max(key_lo, kk)
    ambiguous = False
    tp = np.float32(top_p)
    if tp < np.float32(1.0):
        kept = keys >= key_lo
        w = (np.exp((x[kept] - mx).astype(np.float32)).astype(np.float32) * np.float32(4294967296.0)).astype(np.uint64)
        total = int(w.sum(dtype=np.uint64))
        target = int(np.ceil(np.float64(tp) * np.float64(total)))
        kk = keys[kept]
        order = np.argsort(kk)[::-1]
        ks, ws = kk[order], w[order].astype(np.float64)
        uniq, first = np.unique(ks[::-1], return_index=True)  # ascending unique keys
        # mass per unique key, from the top
        mass = {}
        for key, wt in zip(ks, ws):
            mass[key] = mass.get(key, 0.0) + wt
        cum = 0.0
        tau = ks[0]
        for key in sorted(mass, reverse=True):
            if cum + mass[key] >= target:
                tau = key
                if abs(cum + mass[key] - target) <= 1e-6 * total or abs(cum - target) <= 1e-6 * total:
                    ambiguous = True
                break
            cum += mass[key]
        key_lo = max(key_lo, tau)
    kept = keys >= key_lo
    z = np.exp((x[kept] - mx).astype(np.float32)).astype(np.float64).sum()
    idx = np.nonzero(kept)[0]
    if greedy:
        score = x[idx]
    else:
        score = (x[idx] - log_exp_variates(seed, step, v)[idx]).astype(np.float32)
    tok = int(idx[np.argmax(score)])  # argmax returns the first (lowest index) maximum
    logprob = float(np.float64(x[tok] - mx) - np.log(z))
    return tok, logprob, kept, ambiguous
