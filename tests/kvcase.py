"""Shared helpers for the parity tests: seeded inputs, host<->device copies, tolerances."""

from __future__ import annotations

import numpy as np
import torch

from oracle import paged
from wavelet_amd import synth

# Attention tolerance against the float64 oracle (bf16 output of a bf16/fp8 KV path):
# max |got - ref| <= ATOL outright, elementwise |got - ref| <= ATOL + RTOL * |ref|
# (allclose), and in aggregate ||got - ref||_2 / ||ref||_2 <= RTOL.
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


def check_attention(got: np.ndarray, ref: np.ndarray, what: str, abs_bound: float = ATOL) -> tuple[float, float]:
    """Assert the bar above; returns (max abs error, relative L2 error).

    ``abs_bound`` replaces ATOL in the outright max-abs check only for inputs
    deliberately scaled past N(0, 1) (the bf16 output's own rounding grows with
    the output's magnitude: half an ulp of a value near 16 is 0.03)."""
    err_abs, err_rel = paged.max_abs_and_rel(got, ref)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert err_abs <= abs_bound, f"{what}: max |got-ref| {err_abs:.3e} > {abs_bound}"
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    excess = np.abs(g - r) - (ATOL + RTOL * np.abs(r))
    worst = np.unravel_index(np.argmax(excess), excess.shape) if excess.size else ()
    assert not excess.size or excess.max() <= 0, (
        f"{what}: |got-ref| exceeds {ATOL} + {RTOL}*|ref| at {worst}: got {g[worst]:.5f} ref {r[worst]:.5f}")
    assert err_rel <= RTOL, f"{what}: rel L2 err {err_rel:.3e} > {RTOL}"
    return err_abs, err_rel


# ---------------------------------------------------------------------------
# Guard pads: a device tensor placed inside a larger buffer whose margins hold a
# poison pattern (NaN for float data, the e4m3 NaN code 0x7F for fp8 codes), so
# that a write past either end of the tensor shows up as a changed pad.

PAD = 4096  # elements each side; a multiple of 16 bytes for every dtype used here

_POISON = {torch.bfloat16: (torch.int16, 0x7FC0), torch.uint8: (torch.uint8, 0x7F),
           torch.float32: (torch.int32, 0x7FC00000), torch.int32: (torch.int32, 0x7FC00000),
           torch.int64: (torch.int64, 0x7FF8000000000000)}


class Guarded:
    """A tensor of ``shape`` / ``dtype`` inside a buffer with PAD poisoned elements each side."""

    def __init__(self, shape, dtype, device, fill=None):
        n = int(np.prod(shape)) if len(shape) else 1
        self.buf = torch.empty(n + 2 * PAD, dtype=dtype, device=device)
        self.bits_dtype, self.poison = _POISON[dtype]
        self.buf.view(self.bits_dtype).fill_(self.poison)
        self.t = self.buf[PAD:PAD + n].view(shape)
        if fill is not None:
            self.t.copy_(fill)

    def pads_intact(self) -> bool:
        b = self.buf.view(self.bits_dtype)
        return bool((b[:PAD] == self.poison).all().item()) and bool((b[-PAD:] == self.poison).all().item())


def guard_cache(cache) -> list[Guarded]:
    """Move a PagedKVCache's / MLALatentCache's tensors into guarded buffers (contents kept) and
    point its descriptor at them; returns the guards to check after each launch."""
    guards = []
    names = ("latent",) if hasattr(cache, "latent") else ("k", "v", "k_scale", "v_scale")
    for name in names:
        t = getattr(cache, name)
        if t is None:
            continue
        g = Guarded(tuple(t.shape), t.dtype, t.device, fill=t)
        setattr(cache, name, g.t)
        setattr(cache._desc, name, g.t.data_ptr())
        guards.append(g)
    return guards


def guarded_workspace(device, nbytes: int) -> Guarded:
    """Make the library's per-stream decode workspace exactly ``nbytes`` long inside a guarded
    buffer, so a partial written past the size the library asked for shows up in a pad."""
    from wavelet_amd import attention

    g = Guarded((nbytes,), torch.uint8, device)
    attention._workspaces[attention._key(device)] = g.t
    return g


def assert_guards(guards, what: str) -> None:
    torch.cuda.synchronize()
    for i, g in enumerate(guards):
        assert g.pads_intact(), f"{what}: guard pad {i} around a {tuple(g.t.shape)} tensor was written"
