"""SUBS parameterization and one ancestral sampling step of BD3-LM, on the
CPU. Test infrastructure only (see oracle/__init__.py).

Restates:
* subs_parameterization (model/subs.py:11-43) with the reference's
  log_softmax (model/modules.py:791-799), in the dtypes it runs in under
  bf16 autocast: bf16 logits + bf16 bias (NEG_INF = -1e6 at [MASK]), the
  max and the shift in bf16, exp / sum / log in fp32 (autocast runs them in
  fp32), the final subtraction in fp32; carry-over rows one-hot (0 at x_t,
  NEG_INF elsewhere). fp32 logits run everything in fp32;
* the sampler's step (sample/sampler.py:110-122) and sample_categorical
  (:11-34): q = double(exp(log_probs)) * (1 - s/t), q[mask] = s/t,
  new = argmax(q / (EPS - log(u + EPS))), block = where(block != mask, block, new);
* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11; Random123's philox4x32
  with 10 rounds) and the library's mapping of its output to float64
  uniforms: element e = r * vocab + i uses words (0, 1) (e even) or (2, 3)
  (e odd) of the block with counter {e/2 lo, e/2 hi, offset lo, offset hi}
  and key {seed lo, seed hi}, as (bits >> 11) * 2^-53.
"""
from __future__ import annotations

import numpy as np
import torch

NEG_INF = -1e6
EPS = 1e-10

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_LO = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """ctr (N, 4) uint32, key (N, 2) or (2,) uint32 -> (N, 4) uint32."""
    c = np.array(ctr, dtype=np.uint32, copy=True).reshape(-1, 4)
    k = np.broadcast_to(np.asarray(key, dtype=np.uint32), (c.shape[0], 2)).copy()
    for _ in range(10):
        p0 = _M0 * c[:, 0].astype(np.uint64)
        p1 = _M1 * c[:, 2].astype(np.uint64)
        n0 = (p1 >> np.uint64(32)).astype(np.uint32) ^ c[:, 1] ^ k[:, 0]
        n2 = (p0 >> np.uint64(32)).astype(np.uint32) ^ c[:, 3] ^ k[:, 1]
        c = np.stack([n0, (p1 & _LO).astype(np.uint32), n2, (p0 & _LO).astype(np.uint32)], axis=1)
        k[:, 0] += _W0
        k[:, 1] += _W1
    return c


def philox_uniforms(seed: int, offset: int, rows: int, vocab: int) -> np.ndarray:
    """(rows, vocab) float64 uniforms of the library's Philox mapping."""
    e = np.arange(rows * vocab, dtype=np.uint64)
    pair = e >> np.uint64(1)
    ctr = np.stack([(pair & _LO).astype(np.uint32), (pair >> np.uint64(32)).astype(np.uint32),
                    np.full(e.shape, offset & 0xFFFFFFFF, dtype=np.uint32),
                    np.full(e.shape, (offset >> 32) & 0xFFFFFFFF, dtype=np.uint32)], axis=1)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    w = philox4x32_10(ctr, key)
    odd = (e & np.uint64(1)).astype(bool)
    lo = np.where(odd, w[:, 2], w[:, 0]).astype(np.uint64)
    hi = np.where(odd, w[:, 3], w[:, 1]).astype(np.uint64)
    bits = (hi << np.uint64(32)) | lo
    return ((bits >> np.uint64(11)).astype(np.float64) * 2.0 ** -53).reshape(rows, vocab)


def subs_log_probs(logits: torch.Tensor, xt: torch.Tensor, mask_index: int) -> torch.Tensor:
    """log x_theta (rows, vocab) fp32 for bf16 or fp32 logits (model/subs.py:11-43)."""
    bias = torch.zeros(logits.shape[-1], dtype=logits.dtype)
    bias[mask_index] = NEG_INF
    x = logits + bias                                   # logits dtype
    shifted = x - x.amax(dim=-1, keepdim=True)         # logits dtype
    e = torch.exp(shifted.float())                     # fp32 under autocast
    lp = shifted.float() - torch.log(e.sum(dim=-1, keepdim=True))
    carry = torch.full_like(lp, NEG_INF).scatter(-1, xt.unsqueeze(-1), 0.0)
    unmasked = (xt != mask_index).unsqueeze(-1)
    return torch.where(unmasked, carry, lp)


def sample_step(logits: torch.Tensor, xt: torch.Tensor, mask_index: int, keep: float,
                u: np.ndarray | torch.Tensor) -> torch.Tensor:
    """Next tokens (rows,) int64 of one ancestral step with uniforms u (rows, vocab) float64;
    keep = s / t (sample/sampler.py:110-122, :11-34)."""
    lp = subs_log_probs(logits, xt, mask_index)
    q = torch.exp(lp).double() * (1 - keep)
    q[..., mask_index] = keep
    u = torch.as_tensor(u, dtype=torch.float64)
    gumbel_norm = EPS - torch.log(u + EPS)
    new = torch.argmax(q / gumbel_norm, dim=-1)
    return torch.where(xt != mask_index, xt, new)
