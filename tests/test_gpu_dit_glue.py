"""GPU parity of the fused DiT glue (bd3_ln_modulate, bd3_gate_residual,
bd3_gate_residual_ln_modulate) against oracle/dit.py: the gated residual
bit-exact in every dtype mix; the residual + LayerNorm fusion bit-exact with
the two calls it replaces;
LayerNorm + modulate within the rounding its fp32 row statistics allow
(summation order differs): fp32 results within 1e-5 relative, bf16 results
within one bf16 ulp per rounding of the magnitudes entering the last add, at most 1% of
elements off by any amount."""
from __future__ import annotations

import pytest
import torch

from kernels.dit_glue import gate_residual, ln_modulate
from oracle.dit import gate_residual as ref_gate
from oracle.dit import layer_norm as ref_layer_norm
from oracle.dit import ln_modulate as ref_lnmod

F32, BF = torch.float32, torch.bfloat16


def rnd(shape, dtype, seed, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale + shift).to(dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("xd,md,od", [(F32, BF, F32), (F32, BF, BF), (BF, BF, BF), (BF, F32, F32), (F32, F32, F32)])
# Rows per wave: 4 up to d = 1024, 2 up to 2048, 1 beyond; sequence lengths
# that are not multiples of that put two batch indices in one wave; d = 520
# leaves one lane with a second, last chunk.
@pytest.mark.parametrize("B,S,D", [(2, 37, 768), (1, 5, 64), (8, 256, 768), (2, 9, 2048), (3, 7, 4096),
                                   (2, 11, 520)])
def test_ln_modulate(cuda, xd, md, od, B, S, D):
    print(f"ln_modulate x={xd} mod={md} out={od} shape=({B},{S},{D})", flush=True)
    x = rnd((B, S, D), xd, 1, scale=2.0, shift=0.3)
    w = rnd((D,), F32, 2, scale=0.2, shift=1.0)
    sh, sc = rnd((B, D), md, 3, 0.5), rnd((B, D), md, 4, 0.5)
    want = ref_lnmod(x, w, sh, sc)
    got = ln_modulate(x.to(cuda), w.to(cuda), sh.to(cuda)[:, None], sc.to(cuda)[:, None],
                      out_dtype=od if od != want.dtype else None).cpu()
    assert got.dtype == od
    if od == F32 and xd == F32:
        assert torch.allclose(got, want.float(), rtol=1e-5, atol=1e-5)
    else:
        # A row statistic one fp32 ulp off can move a rounding to bf16 (of y
        # when x is bf16, then of the product and of the sum on the bf16
        # path) by one bf16 ulp each, i.e. at most 2^-7 relative per rounding:
        # within 3 * 2^-7 of the magnitudes entering the last add.
        h = ref_layer_norm(x, w).float()
        mag = (h * (1 + sc.float()[:, None])).abs() + sh.float()[:, None].abs()
        diff = (got.float() - want.to(od).float()).abs()
        assert (diff <= 3 * 2.0 ** -7 * mag + 1e-30).all(), float((diff / (mag + 1e-30)).max())
        assert (diff > 0).float().mean() < 0.01, float((diff > 0).float().mean())


@pytest.mark.gpu
@pytest.mark.parametrize("xd,gd,yd", [(F32, BF, BF), (BF, BF, BF), (F32, F32, F32), (BF, F32, BF)])
@pytest.mark.parametrize("B,S,D", [(3, 50, 768), (2, 7, 520), (1, 3, 64)])
def test_gate_residual_bit_exact(cuda, xd, gd, yd, B, S, D):
    x, g, y = rnd((B, S, D), xd, 5), rnd((B, D), gd, 6), rnd((B, S, D), yd, 7)
    want = ref_gate(x, g, y)
    got = gate_residual(x.to(cuda), g.to(cuda)[:, None], y.to(cuda)).cpu()
    assert got.dtype == want.dtype and torch.equal(got, want)


@pytest.mark.gpu
def test_gate_residual_in_place(cuda):
    x = rnd((2, 16, 64), F32, 8).to(cuda)
    g, y = rnd((2, 64), BF, 9).to(cuda), rnd((2, 16, 64), BF, 10).to(cuda)
    want = ref_gate(x.cpu(), g.cpu(), y.cpu())
    out = gate_residual(x, g, y, out=x)
    assert out.data_ptr() == x.data_ptr() and torch.equal(x.cpu(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("xd,md,yd,od", [(BF, BF, BF, BF), (F32, BF, BF, None), (F32, BF, BF, BF),
                                         (BF, F32, BF, None), (F32, F32, F32, None)])
@pytest.mark.parametrize("B,S,D", [(2, 37, 768), (1, 5, 64), (3, 2, 4096), (2, 9, 2048), (2, 11, 520)])
def test_gate_residual_ln_modulate_matches_two_calls(cuda, xd, md, yd, od, B, S, D):
    """The fused residual + LayerNorm + modulate equals gate_residual followed
    by ln_modulate bit for bit (same kernels' arithmetic, one launch), both
    outputs, including the in-place residual update; vectors sliced from one
    (batch, 6, 1, d) adaLN tensor as the model does."""
    from kernels.dit_glue import gate_residual_ln_modulate
    print(f"gate_residual_ln_modulate x={xd} mod={md} y={yd} out={od} shape=({B},{S},{D})", flush=True)
    x = rnd((B, S, D), xd, 11, scale=2.0, shift=0.3).to(cuda)
    y = rnd((B, S, D), yd, 12).to(cuda)
    ada = rnd((B, 6, 1, D), md, 13, 0.5).to(cuda)
    g, sh, sc = ada[:, 2], ada[:, 3], ada[:, 4]
    w = rnd((D,), F32, 14, scale=0.2, shift=1.0).to(cuda)
    want_x = gate_residual(x, g, y)
    want_h = ln_modulate(want_x, w, sh, sc, out_dtype=od)
    got_x, got_h = gate_residual_ln_modulate(x, g, y, w, sh, sc, out_dtype=od)
    assert got_x.dtype == want_x.dtype and got_h.dtype == want_h.dtype
    assert torch.equal(got_x, want_x) and torch.equal(got_h, want_h)
    if got_x.dtype == x.dtype:  # in place
        x2 = x.clone()
        got_x2, got_h2 = gate_residual_ln_modulate(x2, g, y, w, sh, sc, out_dtype=od, x_out=x2)
        assert got_x2.data_ptr() == x2.data_ptr()
        assert torch.equal(x2, want_x) and torch.equal(got_h2, want_h)
    # gate and the modulation vectors from different adaLN tensors (the last
    # layer's gate with the final layer's shift / scale): batch strides differ
    fin = rnd((B, 2, 1, D), md, 15, 0.5).to(cuda)
    want_h3 = ln_modulate(want_x, w, fin[:, 0], fin[:, 1], out_dtype=od)
    _, got_h3 = gate_residual_ln_modulate(x, g, y, w, fin[:, 0], fin[:, 1], out_dtype=od)
    assert torch.equal(got_h3, want_h3)
