"""Split-KV (FlashDecoding) attention for BD3-LM cached sampling, on MI355X.

Drop-in for the reference's kernels/SplitKVDecodeAttention.py:
`split_kv_decode_attention(q, k, v, block_size)` gives the same result as
block_sparse_decode_attention with the keys split across workgroups; each
split writes a normalised fp32 partial and its LSE, merged with LSE weights.
Adds an optional `n_splits` (default: the reference rule
ceil(kv_len / SPLIT_N), :147). Runs bd3_decode_splitkv in libbd3attn.so.
"""
import torch
from torch import Tensor

from kernels._native import as_kernel_input, check, lib, ptr, stream_of, strides
from kernels.BlockSparseDecodeAttention import (
    _check_decode_inputs, _last_stride_1, block_sparse_decode_attention,
)

# keys per split of the reference's default split rule
SPLIT_N = 256


def split_kv_decode_attention(
    q: Tensor,  # (batch, heads, q_len, head_dim): the last q_len positions
    k: Tensor,  # (batch, heads, kv_len, head_dim)
    v: Tensor,
    block_size: int,
    n_splits: int | None = None,
) -> Tensor:
    """Same result as block_sparse_decode_attention, with the keys split
    across workgroups so a decode step fills the GPU
    (reference: kernels/SplitKVDecodeAttention.py:130-171)."""
    B, H, q_len, D = q.shape
    kv_len = k.shape[2]
    if q_len > 64 and n_splits is None:
        # prefill: many query tiles already fill the GPU (reference :140-142)
        return block_sparse_decode_attention(q, k, v, block_size)
    _check_decode_inputs(q, k, v)
    if n_splits is None:
        n_splits = -(-kv_len // SPLIT_N)
    assert 1 <= n_splits <= kv_len, "n_splits must be in [1, kv_len]"
    q, k, v = as_kernel_input(_last_stride_1(q)), as_kernel_input(k), as_kernel_input(v)
    O = torch.empty((B, H, q_len, D), device=q.device, dtype=q.dtype)
    nbytes = lib().bd3_decode_workspace_bytes(B, H, q_len, kv_len, D, n_splits)
    ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
    check(lib().bd3_decode_splitkv(
        ptr(q), ptr(k), ptr(v), ptr(O), B, H, q_len, kv_len, D, block_size, n_splits,
        strides(q, k, v, O), 1.0 / D ** 0.5, ptr(ws), nbytes, stream_of(q)))
    return O
