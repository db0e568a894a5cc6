"""Pins of oracle/subs.py (CPU): Philox4x32-10 against Random123's published
known-answer vectors, the uniform mapping, the SUBS log-probs against a
float64 log-softmax and their invariants, and the sampling step's
distribution against its closed form (chi-square)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.subs import (EPS, NEG_INF, philox4x32_10, philox_uniforms, sample_step,
                         subs_log_probs)

# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key, output)
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = philox4x32_10(np.array([ctr], dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert tuple(int(x) for x in got[0]) == want


def test_philox_uniform_mapping():
    seed, offset, rows, vocab = 0x123456789ABC, 7, 3, 11  # odd vocab: pairs straddle rows
    u = philox_uniforms(seed, offset, rows, vocab)
    assert u.shape == (rows, vocab) and (u >= 0).all() and (u < 1).all()
    for e in (0, 1, 10, 11, 32):
        p = e // 2
        w = philox4x32_10(np.array([[p, 0, offset, 0]], dtype=np.uint32),
                          np.array([seed & 0xFFFFFFFF, seed >> 32], dtype=np.uint32))[0]
        lo, hi = (int(w[2]), int(w[3])) if e % 2 else (int(w[0]), int(w[1]))
        assert u.reshape(-1)[e] == (((hi << 32) | lo) >> 11) * 2.0 ** -53
    big = philox_uniforms(1, 0, 1, 200_000)
    assert abs(big.mean() - 0.5) < 0.005 and abs(big.var() - 1 / 12) < 0.002
    assert not np.array_equal(philox_uniforms(1, 1, 1, 64), philox_uniforms(1, 0, 1, 64))


# bf16: the shift x - max is rounded to bf16; |x - max| < 32 here, so its
# rounding error is at most half a bf16 ulp at 16..32, 0.0625.
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 0.0626)])
def test_subs_log_probs(dtype, tol):
    rows, vocab, mask = 6, 1000, 999
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(rows, vocab, generator=g) * 3).to(dtype)
    xt = torch.tensor([mask, 5, mask, mask, 17, mask])
    lp = subs_log_probs(logits, xt, mask)
    assert lp.dtype == torch.float32
    ref = torch.log_softmax(logits.double().index_fill(-1, torch.tensor([mask]), -1e300), dim=-1)
    masked = xt == mask
    assert (logits.float().amax(-1) - logits.float().amin(-1) < 32).all()
    # masked rows: normalised over the real tokens, the [MASK] entry pushed far down
    d = (lp[masked, :mask].double() - ref[masked, :mask]).abs().max()
    assert d < tol, float(d)
    assert (lp[masked, mask] < -9e5).all()
    assert torch.allclose(torch.logsumexp(lp[masked].double(), -1), torch.zeros(int(masked.sum()),
                          dtype=torch.float64), atol=1e-5)
    # carry-over rows: one-hot at x_t
    for r in torch.nonzero(~masked).flatten():
        row = lp[r]
        assert row[xt[r]] == 0 and (row[torch.arange(vocab) != xt[r]] == NEG_INF).all()


def test_sample_step_distribution():
    """q_i = p_i (1 - keep) over real tokens, q_mask = keep: chi-square of
    200k draws with independent uniforms."""
    vocab, mask, keep, n = 6, 5, 0.25, 200_000
    p = np.array([0.05, 0.1, 0.15, 0.3, 0.4])
    logits = torch.tensor(np.log(np.append(p, 1.0)), dtype=torch.float32).repeat(n, 1)
    xt = torch.full((n,), mask)
    u = np.random.default_rng(1).random((n, vocab))
    tok = sample_step(logits, xt, mask, keep, u).numpy()
    expect = np.append(p * (1 - keep), keep) * n
    counts = np.bincount(tok, minlength=vocab)
    chi2 = ((counts - expect) ** 2 / expect).sum()
    assert chi2 < 20.5, (chi2, counts, expect)  # 5 d.o.f., p = 0.001


def test_sample_step_carry_and_last_step():
    vocab, mask = 50, 49
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(8, vocab, generator=g)
    xt = torch.tensor([mask, 3, mask, 7, mask, mask, 1, mask])
    u = np.random.default_rng(2).random((8, vocab))
    tok = sample_step(logits, xt, mask, 0.0, u)  # s = 0: every masked token resolves
    assert (tok[xt != mask] == xt[xt != mask]).all()
    assert (tok != mask).all()
    tok1 = sample_step(logits, xt, mask, 1.0 - 1e-12, u)  # s ~ t: masked tokens stay masked
    assert (tok1[xt == mask] == mask).all()
    assert EPS == 1e-10
