"""Shared helpers for the parity tests: seeded inputs, host<->device copies, tolerances."""

from __future__ import annotations

import numpy as np
import torch

from oracle import paged
from wavelet_amd import synth

# Attention tolerance against the float64 oracle (bf16 output of a bf16/fp8 KV path):
# elementwise |got - ref| <= ATOL + RTOL * |ref| (allclose), and in aggregate
# ||got - ref||_2 / ||ref||_2 <= RTOL.
ATOL = 2e-2
RTOL = 1e-2


def to_dev_bits(a: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    """numpy uint16 (bf16 bits) / uint8 (fp8 codes) -> device tensor of `dtype`."""
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(dtype)
    if a.dtype == np.uint8:
        return torch.from_numpy(np.ascontiguousarray(a)).to(device).view(dtype)
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bits_of(t: torch.Tensor) -> np.ndarray:
    """Device bf16 / uint8 tensor -> numpy bit patterns (uint16 / uint8)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.uint8:
        return t.numpy()
    return t.numpy()


def slots_for(w: synth.DecodeWorkload, lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    """Slots of token positions [lo_i, hi_i) of every sequence, sequence-major."""
    out = []
    for i in range(w.batch):
        pos = np.arange(int(lo[i]), int(hi[i]))
        out.append(w.block_tables[i][pos // w.block_size].astype(np.int64) * w.block_size + pos % w.block_size)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def check_attention(got: np.ndarray, ref: np.ndarray, what: str) -> tuple[float, float]:
    err_abs, err_rel = paged.max_abs_and_rel(got, ref)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    excess = np.abs(g - r) - (ATOL + RTOL * np.abs(r))
    worst = np.unravel_index(np.argmax(excess), excess.shape) if excess.size else ()
    assert not excess.size or excess.max() <= 0, (
        f"{what}: |got-ref| exceeds {ATOL} + {RTOL}*|ref| at {worst}: got {g[worst]:.5f} ref {r[worst]:.5f}")
    assert err_rel <= RTOL, f"{what}: rel L2 err {err_rel:.3e} > {RTOL}"
    return err_abs, err_rel
