"""Block-sparse decode attention for BD3-LM sampling, on MI355X.

Drop-in for the reference's kernels/BlockSparseDecodeAttention.py:
`block_sparse_decode_attention(q, k, v, block_size)` attends the last q_len
of kv_len positions block-causally (row i at position kv_len - q_len + i sees
keys j with j // block_size <= position // block_size). Runs bd3_decode in
libbd3attn.so, which picks a key split that fills the GPU (the reference
launches one program per (batch*head, query tile), :132-135; the result is
the same).
"""
import torch
from torch import Tensor

from kernels._native import as_kernel_input, check, lib, ptr, stream_of, strides


def _last_stride_1(x: Tensor) -> Tensor:
    # the kernels need contiguous rows; other strides are fine
    # (reference :113-115)
    return x if x.stride(-1) == 1 else x.contiguous()


def _check_decode_inputs(q: Tensor, k: Tensor, v: Tensor) -> None:
    B, H, q_len, D = q.shape
    kv_len = k.shape[2]
    assert q_len <= kv_len, "queries are the last q_len key positions"
    assert q.is_cuda, "inputs must be on CUDA"
    assert k.shape == v.shape and k.shape[:2] == (B, H) and k.shape[3] == D, "k, v must match q"
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16, "bf16 inputs only"
    assert D == 64, "head_dim must be 64"


def block_sparse_decode_attention(
    q: Tensor,  # (batch, heads, q_len, head_dim): the last q_len positions
    k: Tensor,  # (batch, heads, kv_len, head_dim)
    v: Tensor,
    block_size: int,
) -> Tensor:
    """Block-causal attention of the last q_len positions over all kv_len
    keys (reference: kernels/BlockSparseDecodeAttention.py:118-148)."""
    _check_decode_inputs(q, k, v)
    B, H, q_len, D = q.shape
    kv_len = k.shape[2]
    q, k, v = as_kernel_input(_last_stride_1(q)), as_kernel_input(k), as_kernel_input(v)
    O = torch.empty((B, H, q_len, D), device=q.device, dtype=q.dtype)
    nbytes = lib().bd3_decode_workspace_bytes(B, H, q_len, kv_len, D, 0)
    ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
    check(lib().bd3_decode(
        ptr(q), ptr(k), ptr(v), ptr(O), B, H, q_len, kv_len, D, block_size,
        strides(q, k, v, O), 1.0 / D ** 0.5, ptr(ws), nbytes, stream_of(q)))
    return O
