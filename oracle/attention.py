"""Eager masked attention on the CPU: the fp32 oracle of the BD3-LM attention
path. Test infrastructure only (see oracle/__init__.py).

Restates model/modules.py:728-771 (softmax + scaled_dot_product_attention):
the logits are formed in fp32 (inputs upcast before the product), masked
entries become -inf, the softmax subtracts the row max, the probabilities are
cast to v's dtype and multiplied by v. Feed it bf16-rounded inputs upcast to
fp32 so a comparison measures the kernel, not the input rounding.
"""
from __future__ import annotations

import torch
from torch import Tensor

from oracle.mask import block_diff_mask, decode_mask


def softmax(x: Tensor, dim: int = -1) -> Tensor:
    """Numerically stable softmax (model/modules.py:728-735)."""
    z = x - x.amax(dim=dim, keepdim=True)
    exp_z = torch.exp(z)
    return exp_z / exp_z.sum(dim=dim, keepdim=True)


def eager_attention(q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None = None,
                    logits_dtype: torch.dtype = torch.float32) -> Tensor:
    """softmax(Q K^T / sqrt(d) + M) V (model/modules.py:738-771).
    A row with every key masked yields NaN, as in the reference (:751-752).
    The logits are fp32 as in the reference; `logits_dtype=torch.float64`
    lifts them for finite-difference checks of the oracle itself."""
    scale = 1.0 / (q.shape[-1] ** 0.5)
    scores = torch.matmul(q.to(logits_dtype), k.to(logits_dtype).transpose(-1, -2)) * scale
    if mask is not None:
        scores = torch.where(mask, scores, -torch.inf)
    probabilities = softmax(scores, dim=-1).to(dtype=v.dtype)
    return torch.matmul(probabilities, v)


def masked_lse(q: Tensor, k: Tensor, mask: Tensor,
               logits_dtype: torch.dtype = torch.float32) -> Tensor:
    """Natural-log logsumexp of the masked scaled logits per row: the L the
    reference's forward kernel stores (L = m + log l,
    kernels/BlockSparseFlashAttention.py:169-172)."""
    scale = 1.0 / (q.shape[-1] ** 0.5)
    scores = torch.matmul(q.to(logits_dtype), k.to(logits_dtype).transpose(-1, -2)) * scale
    scores = torch.where(mask, scores, -torch.inf)
    return torch.logsumexp(scores, dim=-1)


def train_mask(n: int, block_size: int) -> Tensor:
    return torch.from_numpy(block_diff_mask(n, block_size))


def bd3_attention(q: Tensor, k: Tensor, v: Tensor, block_size: int,
                  chunk: int | None = None,
                  logits_dtype: torch.dtype = torch.float32) -> tuple[Tensor, Tensor]:
    """(O, lse) of BD3-LM training attention over cat(x_t, x_0): the eager
    path with block_diff_mask (model/bd3lm.py:10-52, model/modules.py:738-771).
    `chunk` processes that many (b, h) slices at a time (same math, bounded
    memory)."""
    B, H, S, D = q.shape
    mask = train_mask(S // 2, block_size)
    if chunk is None:
        return (eager_attention(q, k, v, mask, logits_dtype),
                masked_lse(q, k, mask, logits_dtype))
    qf, kf, vf = (t.reshape(B * H, S, D) for t in (q, k, v))
    outs, lses = [], []
    for i in range(0, B * H, chunk):
        sl = slice(i, i + chunk)
        outs.append(eager_attention(qf[sl], kf[sl], vf[sl], mask, logits_dtype))
        lses.append(masked_lse(qf[sl], kf[sl], mask, logits_dtype))
    return torch.cat(outs).reshape(B, H, S, D), torch.cat(lses).reshape(B, H, S)


def bd3_attention_grads(q: Tensor, k: Tensor, v: Tensor, dout: Tensor, block_size: int,
                        chunk: int | None = None,
                        logits_dtype: torch.dtype = torch.float32
                        ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(O, dQ, dK, dV) of the eager path under autograd, in the inputs' dtype
    (use fp32 or fp64 inputs). The reference's training step differentiates
    exactly this when the "custom" backend is installed."""
    B, H, S, D = q.shape
    mask = train_mask(S // 2, block_size)

    def one(qs, ks, vs, ds):
        qs, ks, vs = (t.detach().clone().requires_grad_(True) for t in (qs, ks, vs))
        o = eager_attention(qs, ks, vs, mask, logits_dtype)
        dq, dk, dv = torch.autograd.grad(o, (qs, ks, vs), ds)
        return o.detach(), dq, dk, dv

    if chunk is None:
        return one(q, k, v, dout)
    flat = [t.reshape(B * H, S, D) for t in (q, k, v, dout)]
    parts = [one(*(t[i:i + chunk] for t in flat)) for i in range(0, B * H, chunk)]
    return tuple(torch.cat([p[j] for p in parts]).reshape(B, H, S, D) for j in range(4))


def bd3_attention_grads_rows(q: Tensor, k: Tensor, v: Tensor, dout: Tensor, block_size: int,
                             rows: int = 1024, delta_factor: float = 1.0
                             ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(O, lse, dQ, dK, dV) of one (b, h) slice (tensors (S, d), fp32), the
    same values as bd3_attention / bd3_attention_grads with memory bounded to
    `rows` x S scores at a time: for long sequences (2n = 8192, 16384), where
    the dense autograd graph holds several S x S fp32 intermediates.

    Written out from the eager path's closed-form gradients (the reference
    differentiates model/modules.py:738-771 with autograd): per row block,
    P = softmax(S * scale + M) (M from model/bd3lm.py:10-52), O = P V cast as
    the reference casts P to v's dtype, Delta = rowsum(dO o O),
    dP = dO V^T, dS = P o (dP - Delta), dQ = scale dS K; dK += scale dS^T Q and
    dV += P^T dO summed over the row blocks. `delta_factor` multiplies Delta:
    1 is the algorithm; tests pass another value to plant a mistake and show
    that a property test catches it."""
    S, D = q.shape
    n = S // 2
    scale = 1.0 / D ** 0.5
    mask = train_mask(n, block_size)
    o = torch.empty_like(q)
    lse = torch.empty(S, dtype=q.dtype)
    dq = torch.empty_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    for r0 in range(0, S, rows):
        sl = slice(r0, min(r0 + rows, S))
        s = torch.matmul(q[sl], k.transpose(-1, -2)) * scale
        s = torch.where(mask[sl], s, -torch.inf)
        lse[sl] = torch.logsumexp(s, dim=-1)
        p = softmax(s, dim=-1)
        o[sl] = torch.matmul(p.to(v.dtype), v)
        delta = (dout[sl] * o[sl]).sum(-1, keepdim=True) * delta_factor
        ds = p * (torch.matmul(dout[sl], v.transpose(-1, -2)) - delta)
        dq[sl] = torch.matmul(ds, k) * scale
        dk += torch.matmul(ds.transpose(-1, -2), q[sl]) * scale
        dv += torch.matmul(p.transpose(-1, -2), dout[sl])
    return o, lse, dq, dk, dv


def decode_attention(q: Tensor, k: Tensor, v: Tensor, block_size: int,
                     logits_dtype: torch.dtype = torch.float32) -> Tensor:
    """Block-causal attention of the last q_len positions over kv_len keys
    (kernels/BlockSparseDecodeAttention.py:118-148 semantics; mask
    oracle.mask.decode_mask)."""
    mask = torch.from_numpy(decode_mask(q.shape[-2], k.shape[-2], block_size))
    return eager_attention(q, k, v, mask, logits_dtype)


def split_partials(q: Tensor, k: Tensor, v: Tensor, block_size: int,
                   bounds: list[tuple[int, int]]) -> tuple[Tensor, Tensor]:
    """Per-split normalised partial outputs and natural-log LSEs over the key
    ranges `bounds` (kernels/SplitKVDecodeAttention.py:55-87: each split runs
    the online softmax over its keys and stores output / l and m + log l)."""
    q_len, kv_len = q.shape[-2], k.shape[-2]
    mask = torch.from_numpy(decode_mask(q_len, kv_len, block_size))
    scale = 1.0 / (q.shape[-1] ** 0.5)
    scores = torch.matmul(q.float(), k.float().transpose(-1, -2)) * scale
    scores = torch.where(mask, scores, -torch.inf)
    parts, lses = [], []
    for lo, hi in bounds:
        s = scores[..., lo:hi]
        lse = torch.logsumexp(s, dim=-1)
        p = torch.exp(s - lse[..., None].clamp_min(-1e30))
        p = torch.nan_to_num(p, nan=0.0)
        parts.append(torch.matmul(p, v[..., lo:hi, :].float()))
        lses.append(lse)
    return torch.stack(parts, dim=-3), torch.stack(lses, dim=-2)


def split_merge(parts: Tensor, lses: Tensor) -> Tensor:
    """LSE-weighted merge of split partials
    (kernels/SplitKVDecodeAttention.py:109-127):
    O = sum_s e^(lse_s - m) part_s / sum_s e^(lse_s - m), m = max_s lse_s.
    parts: (..., n_splits, q_len, d); lses: (..., n_splits, q_len)."""
    m = lses.amax(dim=-2, keepdim=True)
    w = torch.exp(lses - m)
    return (w[..., None] * parts).sum(dim=-3) / w.sum(dim=-2)[..., None]


def useful_flops_fwd(batch: int, heads: int, n: int, block_size: int, d: int = 64) -> int:
    """Useful forward FLOPs 4*d*B*H*(n^2 + n*bs): two products (QK^T, PV) of
    2*d FLOPs per live pair (the reference's count restricted to unmasked
    pairs; bench/attention_bench.py:89)."""
    return 4 * d * batch * heads * (n * n + n * block_size)


def bf16_round(t: Tensor) -> Tensor:
    """Round to bf16 and back to fp32 (the kernels' input precision)."""
    return t.to(torch.bfloat16).to(torch.float32)


def seeded_normal(shape, seed: int, count: int) -> list[Tensor]:
    """`count` N(0,1) fp32 tensors drawn in order from one CPU generator."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float32) for _ in range(count)]


def rel_frobenius(x: Tensor, ref: Tensor) -> float:
    """||x - ref||_F / ||ref||_F in float64."""
    x, ref = x.double(), ref.double()
    return float(torch.linalg.vector_norm(x - ref) / torch.linalg.vector_norm(ref))


__all__ = [
    "softmax", "eager_attention", "masked_lse", "train_mask", "bd3_attention",
    "bd3_attention_grads", "decode_attention", "split_partials", "split_merge",
    "useful_flops_fwd", "bf16_round", "seeded_normal", "rel_frobenius",
]
