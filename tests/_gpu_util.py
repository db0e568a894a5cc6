"""Shared helpers of the GPU parity tests (inputs, C-ABI calls)."""
from __future__ import annotations

import ctypes

import torch

from kernels._native import check, lib, ptr, stream_of, strides
from oracle.attention import bf16_round, seeded_normal

D = 64


def train_inputs(B, H, n, seed=0, count=4, q_scale=1.0):
    """q, k, v[, dO] ~ N(0,1) drawn in that order from `seed` (fp32 CPU),
    q optionally pre-scaled (config 0 scales q by 1/sqrt(d))."""
    ts = seeded_normal((B, H, 2 * n, D), seed, count)
    ts[0] = ts[0] * q_scale
    return [bf16_round(t) for t in ts]


def key_shift_inputs(B, H, n, seed=0):
    """q, v, dO ~ N(0,1) rounded to bf16; keys on a 1/16 grid in [-4, 4] and
    one shift vector c per (b, h) on the same grid in [-2, 2], so that k and
    k + c are both exact in bf16 (every value a multiple of 1/16 below 8 in
    magnitude). Returns q, k, v, dO (B, H, 2n, 64) and c (B, H, 1, 64)."""
    g = torch.Generator().manual_seed(seed)
    q, v, do = (bf16_round(torch.randn(B, H, 2 * n, D, generator=g)) for _ in range(3))
    k = (torch.randn(B, H, 2 * n, D, generator=g) * 16).round().clamp(-64, 64) / 16
    c = (torch.randn(B, H, 1, D, generator=g) * 8).round().clamp(-32, 32) / 16
    assert torch.equal(bf16_round(k), k) and torch.equal(bf16_round(k + c), k + c)
    return q, k, v, do, c


def to_dev(ts, device):
    return [t.to(device=device, dtype=torch.bfloat16) for t in ts]


def fwd_capi(q, k, v, block_size):
    """O and lse straight through bd3_attn_fwd."""
    B, H, S, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), device=q.device, dtype=torch.float32)
    check(lib().bd3_attn_fwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, S // 2, D, block_size,
                             strides(q, k, v, o), 1.0 / D ** 0.5, stream_of(q)))
    return o, lse


def bwd_capi(q, k, v, o, dout, lse, block_size):
    B, H, S, _ = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    nbytes = lib().bd3_attn_bwd_workspace_bytes(B, H, S // 2, D)
    ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    check(lib().bd3_attn_bwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(dout), ptr(lse), ptr(dq), ptr(dk),
                             ptr(dv), ptr(ws), nbytes, B, H, S // 2, D, block_size,
                             strides(q, k, v, o, dout, dq, dk, dv), 1.0 / D ** 0.5, stream_of(q)))
    return dq, dk, dv


def splitkv_capi(q, k, v, block_size, n_splits):
    B, H, q_len, _ = q.shape
    kv_len = k.shape[2]
    o = torch.empty_like(q)
    nbytes = lib().bd3_decode_workspace_bytes(B, H, q_len, kv_len, D, n_splits)
    ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
    check(lib().bd3_decode_splitkv(ptr(q), ptr(k), ptr(v), ptr(o), B, H, q_len, kv_len, D, block_size,
                                   n_splits, strides(q, k, v, o), 1.0 / D ** 0.5, ptr(ws), nbytes,
                                   stream_of(q)))
    return o


def max_abs(a, b) -> float:
    return float((a.double().cpu() - b.double().cpu()).abs().max())
