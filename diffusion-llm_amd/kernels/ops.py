"""torch.library custom ops over libbd3attn.so, with fake kernels.

The reference's sampling ladder wraps its callers in
torch.compile(dynamic=True) (inference/generate.py:39-61). A ctypes call is
opaque to the compiler, so each entry point is registered as a custom op
with a fake (shape-only) kernel: the compiler traces through it without a
graph break, and the real kernel runs at execution time. The training op
carries its backward (register_autograd).

    torch.ops.bd3.attn_fwd(q, k, v, block_size) -> (O, L)      differentiable in q, k, v
    torch.ops.bd3.attn_bwd(q, k, v, O, L, dO, block_size) -> (dQ, dK, dV)
    torch.ops.bd3.decode(q, k, v, block_size, n_splits) -> O   n_splits 0: the library's
        automatic split (bd3_decode), -1: the reference's split rule (ceil(kv_len / 256),
        split_kv_decode_attention's default), > 0: that many splits
"""
from __future__ import annotations

import torch
from torch import Tensor

from kernels._native import as_kernel_input, check, lib, ptr, stream_of, strides

D = 64


def _check_train(q: Tensor, k: Tensor, v: Tensor) -> None:
    B, H, S, Dh = q.shape
    assert q.is_cuda, "inputs must be on CUDA"
    assert q.shape == k.shape == v.shape, "q, k, v must match"
    assert S % 2 == 0 and (S // 2) % 128 == 0, "sequence must be 2n with n a multiple of 128"
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16 and Dh == D, "bf16 inputs with head_dim 64"


@torch.library.custom_op("bd3::attn_fwd", mutates_args=())
def attn_fwd(q: Tensor, k: Tensor, v: Tensor, block_size: int) -> tuple[Tensor, Tensor]:
    """BD3-LM training attention forward: O and the natural-log L per row
    (kernels/BlockSparseFlashAttention.py:465-506)."""
    _check_train(q, k, v)
    B, H, S, _ = q.shape
    q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
    o = q.new_empty((B, H, S, D))
    lse = q.new_empty((B, H, S), dtype=torch.float32)
    check(lib().bd3_attn_fwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, S // 2, D, block_size,
                             strides(q, k, v, o), 1.0 / D ** 0.5, stream_of(q)))
    return o, lse


@attn_fwd.register_fake
def _attn_fwd_fake(q, k, v, block_size):
    B, H, S, _ = q.shape
    return q.new_empty((B, H, S, D)), q.new_empty((B, H, S), dtype=torch.float32)


@torch.library.custom_op("bd3::attn_bwd", mutates_args=())
def attn_bwd(q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, dout: Tensor,
             block_size: int) -> tuple[Tensor, Tensor, Tensor]:
    """dQ, dK, dV (kernels/BlockSparseFlashAttention.py:508-562)."""
    B, H, S, _ = q.shape
    n = S // 2
    assert n % block_size == 0, "n must be a multiple of block_size"
    q, k, v, o = (as_kernel_input(t) for t in (q, k, v, o))
    dout = as_kernel_input(dout.to(q.dtype))
    lse = lse.contiguous()
    dq, dk, dv = (q.new_empty((B, H, S, D)) for _ in range(3))
    nbytes = lib().bd3_attn_bwd_workspace_bytes(B, H, n, D)
    ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    check(lib().bd3_attn_bwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(dout), ptr(lse), ptr(dq), ptr(dk), ptr(dv),
                             ptr(ws), nbytes, B, H, n, D, block_size, strides(q, k, v, o, dout, dq, dk, dv),
                             1.0 / D ** 0.5, stream_of(q)))
    return dq, dk, dv


@attn_bwd.register_fake
def _attn_bwd_fake(q, k, v, o, lse, dout, block_size):
    B, H, S, _ = q.shape
    return tuple(q.new_empty((B, H, S, D)) for _ in range(3))


def _fwd_setup_context(ctx, inputs, output):
    q, k, v, block_size = inputs
    o, lse = output
    ctx.save_for_backward(q, k, v, o, lse)
    ctx.block_size = block_size


def _fwd_backward(ctx, d_o, d_lse):
    q, k, v, o, lse = ctx.saved_tensors
    dq, dk, dv = attn_bwd(q, k, v, o, lse, d_o, ctx.block_size)
    return dq, dk, dv, None


attn_fwd.register_autograd(_fwd_backward, setup_context=_fwd_setup_context)


@torch.library.custom_op("bd3::decode", mutates_args=())
def decode(q: Tensor, k: Tensor, v: Tensor, block_size: int, n_splits: int) -> Tensor:
    """Block-causal decode of the last q_len positions
    (kernels/BlockSparseDecodeAttention.py:118-148); n_splits > 0 runs the
    split-KV form (kernels/SplitKVDecodeAttention.py:130-171)."""
    from kernels.BlockSparseDecodeAttention import block_sparse_decode_attention
    from kernels.SplitKVDecodeAttention import split_kv_decode_attention
    if n_splits == 0:
        return block_sparse_decode_attention(q, k, v, block_size)
    return split_kv_decode_attention(q, k, v, block_size, n_splits=None if n_splits < 0 else n_splits)


@decode.register_fake
def _decode_fake(q, k, v, block_size, n_splits):
    return q.new_empty(q.shape)
