"""Token sampling: the step after the last layer's decode.

What the engine records per generated token -- the token id, its processed
logprob and the sampling mask (``llm.generate`` with
``logprobs_mode="processed_logprobs"`` and ``return_sampling_mask``,
wavelet/inference/engine.py:795-805; consumed by
``extract_vllm_generation_logprobs`` / ``extract_vllm_sampling_mask``,
engine.py:187-256) -- from logits and the per-request ``SamplingParams`` of
``vllm_sampling_kwargs`` (engine.py:69-90): temperature, top_p, top_k, min_p,
repetition_penalty, seed.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .cache import _require_cuda, _stream


# Ranges a scalar parameter must lie in (the reference's sampling config:
# configs/config.py:854-859); per-row tensors are not read back (that would
# synchronise): the kernel keeps at least the row's maximum whatever min_p is.
_RANGES = {
    "temperature": (lambda x: x >= 0.0, ">= 0"),
    "top_p": (lambda x: 0.0 < x <= 1.0, "in (0, 1]"),
    "min_p": (lambda x: 0.0 <= x <= 1.0, "in [0, 1]"),
    "repetition_penalty": (lambda x: x > 0.0, "> 0"),
}


def _check_scalar(name: str, v) -> None:
    if v is not None and not isinstance(v, torch.Tensor) and name in _RANGES:
        ok, text = _RANGES[name]
        if not ok(float(v)):
            raise ValueError(f"{name} must be {text} (got {v})")


def _per_row(v, name: str, batch: int, dtype: torch.dtype, device: torch.device):
    if v is None:
        return None
    if isinstance(v, torch.Tensor):
        _require_cuda(v, name, device)
        if v.dim() == 0:
            v = v.reshape(1).expand(batch)
        if tuple(v.shape) != (batch,):
            raise ValueError(f"{name} must have one value per row ({batch})")
        return v.to(dtype).contiguous()
    return torch.full((batch,), v, dtype=dtype, device=device)


def sample(
    logits: torch.Tensor,
    *,
    temperature=None,
    top_k=None,
    top_p=None,
    min_p=None,
    repetition_penalty=None,
    seen: torch.Tensor | None = None,
    seeds: torch.Tensor | None = None,
    step: int = 0,
    return_mask: bool = False,
    out=None,
):
    """Sample one token per row of ``logits [B, V]`` (fp32 or bf16).

    Per-row parameters are scalars or ``[B]`` tensors (``None``: off /
    defaults). ``seen`` is a ``[B, ceil(V/32)]`` int32 bitmap of the tokens the
    repetition penalty applies to (``seen_bitmap`` builds it); ``seeds [B]``
    int64 and ``step`` fix the random stream. Returns ``(tokens [B] int64,
    logprobs [B] fp32, mask, counts)``; ``mask`` is the ``[B, ceil(V/32)]``
    int32 bitmap of the kept set (``mask_token_ids`` lists it) and ``counts``
    its sizes, both ``None`` unless ``return_mask``. ``out`` may hold those four
    outputs, preallocated (mask and counts may be ``None`` without
    ``return_mask``): a serving loop then allocates nothing per step.
    """
    for name, v in (("temperature", temperature), ("top_p", top_p), ("min_p", min_p),
                    ("repetition_penalty", repetition_penalty)):
        _check_scalar(name, v)
    if logits.dim() != 2 or logits.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("logits must be a float32 or bfloat16 [B, V] tensor")
    dev = logits.device
    _require_cuda(logits, "logits", dev)
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    batch, vocab = logits.shape
    words = (vocab + 31) // 32
    if out is None:
        tokens = torch.empty(batch, dtype=torch.int64, device=dev)
        logprobs = torch.empty(batch, dtype=torch.float32, device=dev)
        mask = torch.empty((batch, words), dtype=torch.int32, device=dev) if return_mask else None
        counts = torch.empty(batch, dtype=torch.int32, device=dev) if return_mask else None
    else:
        tokens, logprobs, mask, counts = out
        for x, name, dt, shape in ((tokens, "tokens", torch.int64, (batch,)), (logprobs, "logprobs", torch.float32,
                                   (batch,)), (mask, "mask", torch.int32, (batch, words)),
                                   (counts, "counts", torch.int32, (batch,))):
            if x is None:
                if return_mask and name in ("mask", "counts"):
                    raise ValueError(f"out: {name} is needed with return_mask")
                continue
            _require_cuda(x, f"out {name}", dev)
            if x.dtype != dt or tuple(x.shape) != shape or not x.is_contiguous():
                raise ValueError(f"out: {name} must be a contiguous {dt} tensor of shape {shape}")
        if not return_mask:
            mask = counts = None
    if batch == 0:
        return tokens, logprobs, mask, counts
    t = _per_row(temperature, "temperature", batch, torch.float32, dev)
    k = _per_row(top_k, "top_k", batch, torch.int32, dev)
    p = _per_row(top_p, "top_p", batch, torch.float32, dev)
    mp = _per_row(min_p, "min_p", batch, torch.float32, dev)
    rp = _per_row(repetition_penalty, "repetition_penalty", batch, torch.float32, dev)
    if seen is not None:
        _require_cuda(seen, "seen", dev)
        if seen.dtype != torch.int32 or tuple(seen.shape) != (batch, words):
            raise ValueError(f"seen must be an int32 [{batch}, {words}] bitmap")
        seen = seen.contiguous()
    if seeds is not None:
        _require_cuda(seeds, "seeds", dev)
        if seeds.dtype != torch.int64 or tuple(seeds.shape) != (batch,):
            raise ValueError(f"seeds must be int64 [{batch}]")
        seeds = seeds.contiguous()

    def ptr(x):
        return None if x is None else x.data_ptr()

    rc = _lib.load().wkv_sample(
        logits.data_ptr(), 0 if logits.dtype == torch.float32 else 1, logits.stride(0), batch, vocab, ptr(t), ptr(k),
        ptr(p), ptr(mp), ptr(rp), ptr(seen), ptr(seeds), int(step), tokens.data_ptr(), logprobs.data_ptr(),
        ptr(mask), ptr(counts), _stream(dev))
    _lib.check(rc, "sample")
    return tokens, logprobs, mask, counts


def seen_bitmap(token_lists, vocab: int) -> np.ndarray:
    """``[B, ceil(V/32)]`` int32 bitmap of each row's prompt + output token ids."""
    words = (vocab + 31) // 32
    bits = np.zeros((len(token_lists), words * 32), dtype=bool)
    for r, toks in enumerate(token_lists):
        bits[r, np.asarray(toks, dtype=np.int64)] = True
    return np.packbits(bits.reshape(len(token_lists), words, 32)[:, :, ::-1], axis=-1, bitorder="big").view(
        ">u4").astype(np.uint32).reshape(len(token_lists), words).view(np.int32)


def mask_token_ids(mask_row: np.ndarray, vocab: int) -> list[int]:
    """The token ids of one row of the kept-set bitmap (``sampling_mask.token_ids``)."""
    w = np.asarray(mask_row).view(np.uint32)
    bits = (w[:, None] >> np.arange(32, dtype=np.uint32)[None, :]) & np.uint32(1)
    ids = np.nonzero(bits.reshape(-1))[0]
    return [int(i) for i in ids if i < vocab]
