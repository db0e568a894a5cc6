"""Block-sparse FlashAttention for the BD3-LM training mask, on MI355X.

Drop-in for the reference's kernels/BlockSparseFlashAttention.py: same class,
same `apply(q, k, v, block_size)` signature, same saved tensors (q, k, v, O,
L with L the natural-log logsumexp per row), same assertions. The forward
and backward run in libbd3attn.so (bd3_attn_fwd / bd3_attn_bwd).

Differences from the reference, all documented narrowings or widenings:
  * bf16 inputs only and head_dim 64 (the reference's configuration); other
    dtypes raise AssertionError instead of running a dtype-generic Triton
    kernel.
  * q, k, v with 16-byte aligned rows are read in place (no .contiguous()
    copy of the strided V view the fused QKV split produces).
"""
from typing import Any

import torch
from torch import Tensor

from kernels._native import as_kernel_input, check, lib, ptr, stream_of, strides


class BlockSparseFlashAttention(torch.autograd.Function):
    """Attention under the BD3-LM block diffusion mask
    (reference: kernels/BlockSparseFlashAttention.py:454-562)."""

    # Tile shape of the gfx950 kernels (module-level names kept from the
    # reference, :457-463; values are this implementation's).
    FWD_BLOCK_M, FWD_BLOCK_N = 128, 64
    FWD_NUM_WARPS, FWD_NUM_STAGES = 4, 2
    BWD_DQ_BLOCK_M, BWD_DQ_BLOCK_N = 64, 128
    BWD_DQ_NUM_WARPS, BWD_DQ_NUM_STAGES = 4, 2
    BWD_DKDV_BLOCK_KV, BWD_DKDV_BLOCK_Q = 128, 64
    BWD_DKDV_NUM_WARPS, BWD_DKDV_NUM_STAGES = 4, 2

    @staticmethod
    def forward(ctx: Any, q: Tensor, k: Tensor, v: Tensor, block_size: int) -> Tensor:
        B, H, seq_len, D = q.shape
        assert q.is_cuda, "inputs must be on CUDA"
        assert q.shape == k.shape == v.shape, "q, k, v must match"
        assert seq_len % 2 == 0, "BD3-LM input is cat(x_t, x_0): length 2n"
        n = seq_len // 2
        BLOCK_M = BlockSparseFlashAttention.FWD_BLOCK_M
        assert n % BLOCK_M == 0, f"n = seq_len / 2 must be a multiple of {BLOCK_M}"
        assert q.dtype == k.dtype == v.dtype == torch.bfloat16, "bf16 inputs only"
        assert D == 64, "head_dim must be 64"

        q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
        O = torch.empty((B, H, seq_len, D), device=q.device, dtype=q.dtype)
        L = torch.empty((B, H, seq_len), device=q.device, dtype=torch.float32)
        check(lib().bd3_attn_fwd(
            ptr(q), ptr(k), ptr(v), ptr(O), ptr(L), B, H, n, D, block_size,
            strides(q, k, v, O), 1.0 / D ** 0.5, stream_of(q)))

        ctx.save_for_backward(q, k, v, O, L)
        ctx.block_size = block_size
        return O

    @staticmethod
    def backward(ctx: Any, dO: Tensor):  # type: ignore[override]
        q, k, v, O, L = ctx.saved_tensors
        block_size = ctx.block_size
        B, H, seq_len, D = q.shape
        n = seq_len // 2
        assert n % block_size == 0

        dO = as_kernel_input(dO.to(q.dtype))
        dQ = torch.empty((B, H, seq_len, D), device=q.device, dtype=q.dtype)
        dK = torch.empty_like(dQ)
        dV = torch.empty_like(dQ)
        nbytes = lib().bd3_attn_bwd_workspace_bytes(B, H, n, D)
        ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
        check(lib().bd3_attn_bwd(
            ptr(q), ptr(k), ptr(v), ptr(O), ptr(dO), ptr(L), ptr(dQ), ptr(dK), ptr(dV),
            ptr(ws), nbytes, B, H, n, D, block_size,
            strides(q, k, v, O, dO, dQ, dK, dV), 1.0 / D ** 0.5, stream_of(q)))
        return dQ, dK, dV, None
