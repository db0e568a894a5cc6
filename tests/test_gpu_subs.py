"""GPU parity of the fused SUBS + ancestral sampling step (bd3_subs_sample)
against the CPU restatement of the reference (oracle/subs.py): the drawn
tokens are identical given the same uniforms, both caller-provided and the
kernel's own Philox4x32-10 stream; masked / unmasked rows, bf16 and fp32
logits, odd vocabularies, first and last steps, winners decided below fp32
resolution and exact ties; plus the draw's
distribution on the GPU (chi-square)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from kernels.sampling import PhiloxStream, subs_sample_step
from oracle import subs as orc

VOCAB, MASK = 50258, 50257  # the reference's GPT-2 vocabulary + [MASK]


def make(rows, vocab, mask, dtype, seed, masked_frac=0.75):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(rows, vocab, generator=g) * 4).to(dtype)
    xt = torch.randint(0, vocab - 1, (rows,), generator=g)
    xt[xt >= mask] += 1  # real tokens: every id but [MASK]
    xt[torch.rand(rows, generator=g) < masked_frac] = mask
    return logits, xt


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("keep", [0.0, 0.5, 31 / 32])
def test_given_uniforms_match_oracle(cuda, dtype, keep):
    rows = 64
    print(f"subs_sample given-u dtype={dtype} keep={keep}", flush=True)
    logits, xt = make(rows, VOCAB, MASK, dtype, seed=int(keep * 100) + 1)
    u = torch.rand(rows, VOCAB, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    want = orc.sample_step(logits, xt, MASK, keep, u)
    got = subs_sample_step(logits.to(cuda), xt.to(cuda), MASK, keep, u=u.to(cuda))
    assert torch.equal(got.cpu(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,vocab,mask", [(48, VOCAB, MASK), (37, 1001, 0), (5, 3, 1)])
def test_philox_stream_matches_oracle(cuda, rows, vocab, mask):
    print(f"subs_sample philox rows={rows} vocab={vocab}", flush=True)
    logits, xt = make(rows, vocab, mask, torch.bfloat16, seed=rows)
    gen = PhiloxStream(seed=0xDEADBEEF12345)
    for step in range(3):
        keep = 1 - (step + 1) / 3
        off = gen.offset
        got = subs_sample_step(logits.to(cuda), xt.to(cuda), mask, keep, generator=gen)
        u = orc.philox_uniforms(gen.seed, off, rows, vocab)
        want = orc.sample_step(logits, xt, mask, keep, u)
        assert torch.equal(got.cpu(), want), step
        xt = want


@pytest.mark.gpu
def test_strided_logits_and_block_shape(cuda):
    B, L, V = 2, 16, 4099
    g = torch.Generator().manual_seed(5)
    wide = (torch.randn(B, L, V + 61, generator=g) * 2).to(torch.bfloat16)
    logits = wide[..., :V]
    block = torch.full((B, L), V - 1, dtype=torch.int64)
    block[0, :5] = torch.arange(5)
    u = torch.rand(B, L, V, dtype=torch.float64, generator=g)
    got = subs_sample_step(logits.to(cuda), block.to(cuda), V - 1, 0.25, u=u.to(cuda))
    want = orc.sample_step(logits.reshape(B * L, V), block.reshape(-1), V - 1, 0.25, u.reshape(B * L, V))
    assert got.shape == (B, L) and torch.equal(got.cpu().reshape(-1), want)


@pytest.mark.gpu
def test_distribution_on_gpu(cuda):
    """Philox draws over 200k identical rows follow q (chi-square, 5 d.o.f.)."""
    vocab, mask, keep, n = 6, 5, 0.25, 200_000
    p = np.array([0.05, 0.1, 0.15, 0.3, 0.4])
    logits = torch.tensor(np.log(np.append(p, 1.0)), dtype=torch.float32).repeat(n, 1).to(cuda)
    xt = torch.full((n,), mask, device=cuda)
    tok = subs_sample_step(logits, xt, mask, keep, generator=PhiloxStream(seed=77)).cpu().numpy()
    expect = np.append(p * (1 - keep), keep) * n
    chi2 = ((np.bincount(tok, minlength=vocab) - expect) ** 2 / expect).sum()
    assert chi2 < 20.5, chi2


@pytest.mark.gpu
@pytest.mark.parametrize("vocab,mask", [(VOCAB, MASK), (1001, 0)])
def test_near_ties_resolved_exactly(cuda, vocab, mask):
    """Winners decided below fp32 resolution: the pruning filters (an fp32
    estimate of the Gumbel term for u < 0.999, the 1 - u bound above) must
    let every contender through to the float64 ratio, and exact ties go to
    the first index (torch.argmax)."""
    print(f"subs_sample near ties vocab={vocab}", flush=True)
    rows, keep = 4, 1e-6  # q = 1e-6 for [MASK], (1 - 1e-6) / (vocab - 1) for every real token
    logits = torch.zeros(rows, vocab, dtype=torch.bfloat16)
    xt = torch.full((rows,), mask, dtype=torch.int64)
    u = torch.full((rows, vocab), 0.25, dtype=torch.float64)
    a, b = (mask + 100) % vocab, (mask + 200) % vocab
    u[0, a] = 0.999                                    # the 1 - u branch
    u[0, b] = np.nextafter(0.999, 1.0)                 # one float64 ulp closer to 1: wins
    u[1, a] = 0.9                                      # the fp32-estimate branch
    u[1, b] = 0.9 + 1e-15                              # indistinguishable in fp32: wins
    u[2, b] = 0.95                                     # exact tie: the first index wins
    u[2, a] = 0.95
    u[3, mask] = 1 - 2.0 ** -30                        # [MASK] wins through the 1 - u branch
    want = orc.sample_step(logits, xt, mask, keep, u)
    assert want.tolist() == [b, b, min(a, b), mask]
    got = subs_sample_step(logits.to(cuda), xt.to(cuda), mask, keep, u=u.to(cuda))
    assert torch.equal(got.cpu(), want)
