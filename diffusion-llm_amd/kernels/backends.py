"""Attention-backend registry: the operator seam of the BD3-LM model.

The reference model's attention layer calls a module-level function
`scaled_dot_product_attention(q, k, v, mask=None)` that it resolves by name
at call time (model/modules.py:419), and the reference swaps that function
with `install_attention(name, nvtx, block_size)` (bench/attention.py:117-127).
This module keeps that public surface (the `BACKENDS` names, the
`BLOCK_SIZE_BACKENDS` tuple and `install_attention`'s signature) so a caller
switches over by name, and routes each name to the gfx950 library through the
`torch.ops.bd3` custom ops (kernels/ops.py), which trace under torch.compile
without a graph break.

Backends taking a block size do not read `mask`: each one derives the
visibility rule from the block size and the layout it serves.

    name      layout of (q, k, v)                         rule
    bsfa      training sequence cat(x_t, x_0), length 2n  BD3-LM mask; fwd + bwd
    bsdfa     q = last q_len of the kv_len positions      block-causal; fwd only
    split_kv  as bsdfa                                    as bsdfa, keys cut into
                                                          the reference's 256-key splits
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

# Profiler range names (roctx on ROCm builds), as the reference names them.
FORWARD_RANGE = "attention"
BACKWARD_RANGE = "attention backward"

# split count argument of torch.ops.bd3.decode: 0 = the library's automatic
# count, -1 = the reference's ceil(kv_len / 256) rule
_AUTO_SPLITS, _REFERENCE_SPLITS = 0, -1


def bsfa(q, k, v, mask=None, block_size=None):
    """Training attention over cat(x_t, x_0) under the BD3-LM mask of
    `block_size`; differentiable (bd3_attn_fwd / bd3_attn_bwd)."""
    return torch.ops.bd3.attn_fwd(q, k, v, block_size)[0]


def bsdfa(q, k, v, mask=None, block_size=None):
    """Decode / prefill attention: q holds the last q_len of the kv_len key
    positions, visibility block-causal in `block_size` (bd3_decode, automatic
    split count)."""
    return torch.ops.bd3.decode(q, k, v, block_size, _AUTO_SPLITS)


def split_kv(q, k, v, mask=None, block_size=None):
    """Same result as bsdfa, with the keys cut into ceil(kv_len / 256) splits
    merged by their log-sum-exp (bd3_decode_splitkv)."""
    return torch.ops.bd3.decode(q, k, v, block_size, _REFERENCE_SPLITS)


BACKENDS: dict[str, AttentionFn] = {
    "bsfa": bsfa,
    "bsdfa": bsdfa,
    "split_kv": split_kv,
}
BLOCK_SIZE_BACKENDS = ("bsfa", "bsdfa", "split_kv")


class _RangeEdge(torch.autograd.Function):
    """Passes its tensors through unchanged and marks one edge of the
    attention's profiler ranges on the way.

    Placed at the attention's inputs (`entry=True`) it opens the forward
    range and, when the gradients come back through it, closes the backward
    range; placed at the output it closes the forward range and opens the
    backward one. Autograd runs the two backward edges in the reverse order
    of the forward ones, so the ranges nest."""

    @staticmethod
    def forward(ctx, entry: bool, *xs: Tensor):
        ctx.entry = entry
        if entry:
            torch.cuda.nvtx.range_push(FORWARD_RANGE)
        else:
            torch.cuda.nvtx.range_pop()
        return tuple(x.view_as(x) for x in xs)

    @staticmethod
    def backward(ctx, *grads: Tensor):
        if ctx.entry:
            torch.cuda.nvtx.range_pop()
        else:
            torch.cuda.nvtx.range_push(BACKWARD_RANGE)
        return (None, *grads)


def with_ranges(attention: AttentionFn) -> AttentionFn:
    """`attention` with its forward and backward each inside a profiler range
    (the reference's nvtx=True option, bench/attention.py:107-114)."""

    def ranged(q, k, v, mask=None):
        q, k, v = _RangeEdge.apply(True, q, k, v)
        (o,) = _RangeEdge.apply(False, attention(q, k, v, mask))
        return o

    return ranged


def install_attention(
    name: str,
    nvtx: bool = False,
    block_size: int | None = None,
    module: ModuleType | str = "model.modules",
) -> AttentionFn:
    """Make `module.scaled_dot_product_attention` the backend `name` and
    return what was installed (reference: bench/attention.py:117-127).

    `module` is the model module whose attention layer looks the function up
    (the reference patches its own `model.modules`). A name this registry does
    not hold (e.g. the model's eager "custom") is taken from that module's
    own `BACKENDS`. Block-size backends need `block_size`."""
    mod = importlib.import_module(module) if isinstance(module, str) else module
    attention = BACKENDS.get(name) or getattr(mod, "BACKENDS", {})[name]
    if name in BLOCK_SIZE_BACKENDS:
        assert block_size is not None, f"{name} needs block_size"
        attention = partial(attention, block_size=block_size)
    if nvtx:
        attention = with_ranges(attention)
    mod.scaled_dot_product_attention = attention
    return attention
