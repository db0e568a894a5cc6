"""Pins of oracle/dit.py (CPU): the LayerNorm against torch's own
F.layer_norm (weight only, no bias) and its invariants, modulate and the
gated residual against their identity cases and a float64 evaluation."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle.dit import gate_residual, layer_norm, ln_modulate, modulate


def test_layer_norm_matches_library():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 33, 768, generator=g) * 3 + 1.5
    w = torch.rand(768, generator=g) + 0.5
    got = layer_norm(x, w, 1e-5)
    want = F.layer_norm(x, (768,), weight=w, bias=None, eps=1e-5)
    assert torch.allclose(got, want, atol=2e-5, rtol=1e-5)
    unit = layer_norm(x, torch.ones(768), 0.0).double()
    assert torch.allclose(unit.mean(-1), torch.zeros(4, 33, dtype=torch.float64), atol=1e-5)
    assert torch.allclose(unit.var(-1, correction=0), torch.ones(4, 33, dtype=torch.float64), atol=1e-4)
    assert layer_norm(x.to(torch.bfloat16), w).dtype == torch.bfloat16


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_modulate_and_gate_identities(dtype):
    g = torch.Generator().manual_seed(1)
    h = torch.randn(2, 5, 64, generator=g).to(dtype)
    zero = torch.zeros(2, 64, dtype=dtype)
    assert torch.equal(modulate(h, zero, zero), h)
    assert torch.equal(gate_residual(h, zero, torch.randn(2, 5, 64, generator=g).to(dtype)), h)
    y = torch.randn(2, 5, 64, generator=g).to(dtype)
    assert torch.equal(gate_residual(h, torch.ones(2, 64, dtype=dtype), y), h + y)
    sh, sc = torch.randn(2, 64, generator=g), torch.randn(2, 64, generator=g)
    ref = h.double() * (1 + sc.double()[:, None]) + sh.double()[:, None]
    assert torch.allclose(modulate(h.float(), sh, sc).double(), ref, atol=1e-5, rtol=1e-5)
    out = ln_modulate(h, torch.ones(64, dtype=torch.float32), sh.to(dtype), sc.to(dtype))
    assert out.shape == h.shape
