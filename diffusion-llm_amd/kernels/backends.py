"""Attention-backend registry: the operator seam of the BD3-LM model.

Mirrors the reference's bench/attention.py:51-127. A model module exposes a
global `scaled_dot_product_attention(q, k, v, mask=None)` that its attention
layer looks up by name at call time (model/modules.py:419);
`install_attention(name, block_size=...)` replaces that global with one of
the gfx950 backends below. The block-size backends ignore `mask` and rebuild
the BD3-LM mask from `block_size`, exactly as the reference's do (:51-66):

    bsfa      training layout cat(x_t, x_0), forward + backward
    bsdfa     decode / prefill: last q_len positions, block-causal
    split_kv  bsdfa with the keys split across workgroups
"""
from __future__ import annotations

import importlib
from collections.abc import Callable
from functools import partial
from types import ModuleType

import torch
from torch import Tensor

import kernels.ops  # noqa: F401  (registers torch.ops.bd3.*)

AttentionFn = Callable[..., Tensor]

FORWARD_RANGE = "attention"
BACKWARD_RANGE = "attention backward"


# The backends call the custom ops (kernels/ops.py), so a caller wrapped in
# torch.compile traces them without a graph break.


def bsfa(q, k, v, mask=None, block_size=None):
    """Block-sparse FlashAttention (forward + backward) on the 2n training
    layout; it builds the mask from block_size."""
    return torch.ops.bd3.attn_fwd(q, k, v, block_size)[0]


def bsdfa(q, k, v, mask=None, block_size=None):
    """Block-sparse decode attention (forward only): the last q_len
    positions, block-causal; it builds the mask from block_size."""
    return torch.ops.bd3.decode(q, k, v, block_size, 0)


def split_kv(q, k, v, mask=None, block_size=None):
    """Split-KV decode attention (forward only): bsdfa with the keys split
    across workgroups, for decode steps with few queries (the reference's
    split rule)."""
    return torch.ops.bd3.decode(q, k, v, block_size, -1)


BACKENDS: dict[str, AttentionFn] = {
    "bsfa": bsfa,
    "bsdfa": bsdfa,
    "split_kv": split_kv,
}
# backends that ignore the mask and need the block size instead
BLOCK_SIZE_BACKENDS = ("bsfa", "bsdfa", "split_kv")


class _OpenRange(torch.autograd.Function):
    """Identity on (q, k, v) that opens the forward range (roctx on ROCm)."""

    @staticmethod
    def forward(ctx, q, k, v):
        torch.cuda.nvtx.range_push(FORWARD_RANGE)
        return q.view_as(q), k.view_as(k), v.view_as(v)

    @staticmethod
    def backward(ctx, *grad_outputs):
        torch.cuda.nvtx.range_pop()
        return grad_outputs


class _CloseRange(torch.autograd.Function):
    """Identity on the attention output that closes the forward range."""

    @staticmethod
    def forward(ctx, o):
        torch.cuda.nvtx.range_pop()
        return o.view_as(o)

    @staticmethod
    def backward(ctx, *grad_outputs):
        torch.cuda.nvtx.range_push(BACKWARD_RANGE)
        return grad_outputs


def with_ranges(attention: AttentionFn) -> AttentionFn:
    """Wrap a backend in profiler ranges for both forward and backward
    (reference: with_nvtx, bench/attention.py:107-114)."""

    def annotated(q, k, v, mask=None):
        q, k, v = _OpenRange.apply(q, k, v)
        return _CloseRange.apply(attention(q, k, v, mask))

    return annotated


def install_attention(
    name: str,
    nvtx: bool = False,
    block_size: int | None = None,
    module: ModuleType | str = "model.modules",
) -> AttentionFn:
    """Route every attention layer of `module` through the named backend
    (reference: bench/attention.py:117-127). `module` is the model module
    whose global `scaled_dot_product_attention` the attention layer calls;
    names not registered here (e.g. the model's own eager "custom") are
    looked up on that module. Returns the installed callable."""
    mod = importlib.import_module(module) if isinstance(module, str) else module
    if name in BACKENDS:
        attention = BACKENDS[name]
    else:
        attention = getattr(mod, "BACKENDS", {})[name]
    if name in BLOCK_SIZE_BACKENDS:
        assert block_size is not None, f"{name} needs block_size"
        attention = partial(attention, block_size=block_size)
    installed = with_ranges(attention) if nvtx else attention
    mod.scaled_dot_product_attention = installed
    return installed
