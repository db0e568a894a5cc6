"""The DiT block's elementwise glue around attention, on the CPU. Test
infrastructure only (see oracle/__init__.py).

Restates, with torch CPU ops in the reference's dtypes:
* the weight-only LayerNorm (model/modules.py:243-288): the row upcast to
  fp32, mean and variance (correction 0), rsqrt(var + eps), then
  weight * numerator * inv_std and a cast back to x's dtype;
* modulate (model/modules.py:778-788): h * (1 + scale) + shift, broadcast
  over the sequence, in the promoted dtype of its operands;
* the gated residual of DiTBlock.forward (model/modules.py:560-566):
  x + gate * y.
"""
from __future__ import annotations

import torch
from torch import Tensor


def layer_norm(x: Tensor, weight: Tensor, eps: float = 1e-5) -> Tensor:
    xf = x.to(torch.float32)
    num = xf - xf.mean(dim=-1, keepdim=True)
    inv_std = torch.rsqrt(xf.var(dim=-1, keepdim=True, correction=0) + eps)
    return (weight * num * inv_std).to(dtype=x.dtype)


def modulate(h: Tensor, shift: Tensor, scale: Tensor) -> Tensor:
    """h (batch, seq, d); shift, scale (batch, d)."""
    return h * (1 + scale[:, None, :]) + shift[:, None, :]


def ln_modulate(x: Tensor, weight: Tensor, shift: Tensor, scale: Tensor, eps: float = 1e-5) -> Tensor:
    return modulate(layer_norm(x, weight, eps), shift, scale)


def gate_residual(x: Tensor, gate: Tensor, y: Tensor) -> Tensor:
    """x, y (batch, seq, d); gate (batch, d)."""
    return x + gate[:, None, :] * y
