"""Fused SUBS parameterization + ancestral sampling step for BD3-LM
sampling, on MI355X.

`subs_sample_step(logits, block, mask_index, keep)` returns the block after
one denoising step of sample_bd3lm (sample/sampler.py:110-122): SUBS
log-probs of the raw logits (model/subs.py:11-43), q = exp(log_probs) *
(1 - s/t) with q[mask] = s/t, a Gumbel-max draw with float64 noise
(sample_categorical, :11-34), and masked positions replaced by the draw.
One bd3_subs_sample launch does it without writing any (rows, vocab)
intermediate (the reference materialises the log-probs, the carry tensor,
q, the uniforms and the noise, several of them in float64).

Noise: pass `u` (float64, the shape of the logits; e.g. torch.rand_like's
draw) to reproduce the reference's arithmetic on the same uniforms, or let
the kernel draw them from a counter-based Philox4x32-10 stream
(`PhiloxStream`): same distribution, nothing materialised.
"""
from __future__ import annotations

import threading

import torch
from torch import Tensor

from kernels._native import check, lib, ptr, stream_of


class PhiloxStream:
    """Seed and running offset of the kernel's Philox4x32-10 draws: each
    step takes a fresh offset, so no counter is ever reused."""

    def __init__(self, seed: int | None = None):
        self.seed = int(torch.initial_seed() if seed is None else seed) & (2 ** 64 - 1)
        self.offset = 0
        self._lock = threading.Lock()

    def next_offset(self) -> int:
        with self._lock:
            off = self.offset
            self.offset += 1
            return off


_default_stream: PhiloxStream | None = None


def default_stream() -> PhiloxStream:
    global _default_stream
    if _default_stream is None:
        _default_stream = PhiloxStream()
    return _default_stream


def subs_sample_step(
    logits: Tensor,   # (..., vocab) raw backbone logits, bf16 or fp32
    block: Tensor,    # (...) int64 current tokens ([MASK] where still masked)
    mask_index: int,
    keep: float,      # s / t of this step (0 at the last step)
    u: Tensor | None = None,            # (..., vocab) float64 uniforms in [0, 1), or None
    generator: PhiloxStream | None = None,
) -> Tensor:
    """The block after one ancestral step (a new int64 tensor shaped like `block`)."""
    assert logits.is_cuda and logits.dtype in (torch.bfloat16, torch.float32), \
        "logits must be bf16 or fp32 CUDA tensors"
    assert logits.shape[:-1] == block.shape, "block must match the logits' leading dims"
    assert 0.0 <= keep <= 1.0, "keep = s / t must lie in [0, 1]"
    vocab = logits.shape[-1]
    rows = block.numel()
    lg = logits.reshape(rows, vocab)
    if lg.stride(-1) != 1:
        lg = lg.contiguous()
    xt = block.reshape(rows).to(device=logits.device, dtype=torch.int64).contiguous()
    out = torch.empty_like(xt)
    if u is not None:
        assert u.shape == logits.shape and u.dtype == torch.float64 and u.device == logits.device
        u = u.reshape(rows, vocab).contiguous()
        seed = offset = 0
    else:
        gen = generator or default_stream()
        seed, offset = gen.seed, gen.next_offset()
    check(lib().bd3_subs_sample(ptr(lg), lg.stride(0), 1 if lg.dtype == torch.float32 else 0, ptr(xt),
                                ptr(out), rows, vocab, mask_index, float(keep), ptr(u), seed, offset,
                                stream_of(lg)))
    return out.view(block.shape)
