"""The DiT block's elementwise glue around attention, fused, on MI355X.

`ln_modulate(x, weight, shift, scale)` = modulate(LN(x), shift, scale) of
DiTBlock.forward (model/modules.py:537-568; LayerNorm :243-288, modulate
:778-788) in one pass; `gate_residual(x, gate, y)` = x + gate * y
(:560-566). Both follow the reference's eager dtypes (bf16 ops rounded op by
op, fp32 otherwise); gate_residual is bit-exact, ln_modulate differs from the
eager path only by the fp32 summation order of the row statistics.
Shapes: x, y (batch, seq, d_model); shift, scale, gate (batch, d_model) or
(batch, 1, d_model) (the AdaLN chunks); weight (d_model).
"""
from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from kernels._native import check, lib, ptr, stream_of

_F = {torch.float32: 1, torch.bfloat16: 0}


def _vec(t: Tensor) -> Tensor:
    """(batch, d) view of a (batch, d) or (batch, 1, d) modulation vector."""
    if t.dim() == 3:
        assert t.shape[1] == 1, "modulation vectors broadcast over the sequence"
        t = t[:, 0]
    return _ready(t)


def _ready(t: Tensor) -> Tensor:
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


def ln_modulate(x: Tensor, weight: Tensor, shift: Tensor, scale: Tensor, eps: float = 1e-5,
                out_dtype: torch.dtype | None = None) -> Tensor:
    """modulate(LN(x), shift, scale). The result's dtype is the eager one
    (bf16 when x and the vectors are bf16, else fp32); out_dtype=bf16 rounds
    an fp32 result for the next matmul."""
    assert x.dim() == 3 and x.is_cuda, "x must be (batch, seq, d_model) on CUDA"
    B, S, D = x.shape
    x, weight, shift, scale = _ready(x), _ready(weight), _vec(shift), _vec(scale)
    assert shift.dtype == scale.dtype and shift.shape == scale.shape == (B, D)
    natural = torch.bfloat16 if (x.dtype == torch.bfloat16 and shift.dtype == torch.bfloat16) else torch.float32
    out = torch.empty((B, S, D), device=x.device, dtype=out_dtype or natural)
    st = (ctypes.c_int64 * 5)(x.stride(0), x.stride(1), shift.stride(0), out.stride(0), out.stride(1))
    check(lib().bd3_ln_modulate(ptr(x), _F[x.dtype], ptr(weight), _F[weight.dtype], ptr(shift), ptr(scale),
                                _F[shift.dtype], ptr(out), _F[out.dtype], B, S, D, st, float(eps),
                                stream_of(x)))
    return out


def gate_residual(x: Tensor, gate: Tensor, y: Tensor, out: Tensor | None = None) -> Tensor:
    """x + gate * y in the eager dtypes; `out=x` updates the residual in place."""
    assert x.dim() == 3 and x.shape == y.shape and x.is_cuda
    B, S, D = x.shape
    x, y, gate = _ready(x), _ready(y), _vec(gate)
    bf = x.dtype == gate.dtype == y.dtype == torch.bfloat16
    if out is None:
        out = torch.empty((B, S, D), device=x.device, dtype=torch.bfloat16 if bf else torch.float32)
    assert out.dtype == (torch.bfloat16 if bf else torch.float32) and out.shape == x.shape
    st = (ctypes.c_int64 * 7)(x.stride(0), x.stride(1), gate.stride(0), y.stride(0), y.stride(1),
                              out.stride(0), out.stride(1))
    check(lib().bd3_gate_residual(ptr(x), _F[x.dtype], ptr(gate), _F[gate.dtype], ptr(y), _F[y.dtype],
                                  ptr(out), B, S, D, st, stream_of(x)))
    return out


def gate_residual_ln_modulate(x: Tensor, gate: Tensor, y: Tensor, weight: Tensor, shift: Tensor,
                              scale: Tensor, eps: float = 1e-5, out_dtype: torch.dtype | None = None,
                              x_out: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """(x + gate * y, modulate(LN(x + gate * y), shift, scale)) in one launch,
    bit-exact with gate_residual followed by ln_modulate; `x_out=x` updates
    the residual in place."""
    assert x.dim() == 3 and x.shape == y.shape and x.is_cuda
    B, S, D = x.shape
    x, y, weight = _ready(x), _ready(y), _ready(weight)
    gate, shift, scale = _vec(gate), _vec(shift), _vec(scale)
    assert gate.dtype == shift.dtype == scale.dtype and gate.shape == shift.shape == scale.shape == (B, D)
    if not gate.stride(0) == shift.stride(0) == scale.stride(0):  # one batch stride for the three
        gate, shift, scale = gate.contiguous(), shift.contiguous(), scale.contiguous()
    res = torch.bfloat16 if x.dtype == gate.dtype == y.dtype == torch.bfloat16 else torch.float32
    if x_out is None:
        x_out = torch.empty((B, S, D), device=x.device, dtype=res)
    assert x_out.dtype == res and x_out.shape == x.shape
    natural = torch.bfloat16 if (res == torch.bfloat16 and shift.dtype == torch.bfloat16) else torch.float32
    out = torch.empty((B, S, D), device=x.device, dtype=out_dtype or natural)
    st = (ctypes.c_int64 * 9)(x.stride(0), x.stride(1), gate.stride(0), y.stride(0), y.stride(1),
                              x_out.stride(0), x_out.stride(1), out.stride(0), out.stride(1))
    check(lib().bd3_gate_residual_ln_modulate(ptr(x), _F[x.dtype], ptr(gate), ptr(y), _F[y.dtype], ptr(x_out),
                                              ptr(weight), _F[weight.dtype], ptr(shift), ptr(scale),
                                              _F[shift.dtype], ptr(out), _F[out.dtype], B, S, D, st, float(eps),
                                              stream_of(x)))
    return x_out, out
