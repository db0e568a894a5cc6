"""Pins the attention oracle (oracle/attention.py): brute-force known
answers, special cases that reduce to torch's SDPA, finite-difference
gradients, closed-form backward identities and the split-KV merge."""
import json
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from oracle.attention import (bd3_attention, bd3_attention_grads, bd3_attention_grads_rows,
                              decode_attention, eager_attention, masked_lse, split_merge, split_partials,
                              train_mask, useful_flops_fwd)

GOLDEN = json.loads((Path(__file__).parent / "golden" / "bd3_golden.json").read_text())


@pytest.mark.parametrize("case", GOLDEN["attention"], ids=lambda c: f"n{c['n']}_bs{c['block_size']}")
def test_bruteforce_fixture(case):
    n, bs, d = case["n"], case["block_size"], case["d"]
    shape = (1, 1, 2 * n, d)
    q, k, v = (torch.tensor(case[x], dtype=torch.float64).reshape(shape) for x in "qkv")
    # fp64 path of the same restatement (probabilities cast to v's dtype)
    o = eager_attention(q.double(), k.double(), v.double(), train_mask(n, bs))
    scale = 1 / d ** 0.5
    s = torch.where(train_mask(n, bs), q @ k.transpose(-1, -2) * scale, -torch.inf)
    assert torch.allclose(o.flatten().double(), torch.tensor(case["out"], dtype=torch.float64), atol=1e-6)
    assert torch.allclose(torch.logsumexp(s, -1).flatten(), torch.tensor(case["lse"], dtype=torch.float64),
                          atol=1e-12)
    # the fp32 oracle within fp32 rounding of the brute force
    o32, lse32 = bd3_attention(q.float(), k.float(), v.float(), bs)
    assert torch.allclose(o32.flatten().double(), torch.tensor(case["out"], dtype=torch.float64), atol=1e-5)
    assert torch.allclose(lse32.flatten().double(), torch.tensor(case["lse"], dtype=torch.float64), atol=1e-5)


def rand(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


def test_block_size_n_is_two_sdpa_calls():
    n, d = 32, 16
    q, k, v = (rand(2, 3, 2 * n, d, seed=s) for s in range(3))
    o, _ = bd3_attention(q, k, v, n, logits_dtype=torch.float64)
    ref_noisy = F.scaled_dot_product_attention(q[..., :n, :], k[..., :n, :], v[..., :n, :])
    ref_clean = F.scaled_dot_product_attention(q[..., n:, :], k[..., n:, :], v[..., n:, :])
    assert torch.allclose(o, torch.cat([ref_noisy, ref_clean], dim=-2), atol=1e-12)


def test_block_size_1_clean_half_is_causal_sdpa():
    n, d = 24, 8
    q, k, v = (rand(1, 2, 2 * n, d, seed=s + 10) for s in range(3))
    o, _ = bd3_attention(q, k, v, 1, logits_dtype=torch.float64)
    ref = F.scaled_dot_product_attention(q[..., n:, :], k[..., n:, :], v[..., n:, :], is_causal=True)
    assert torch.allclose(o[..., n:, :], ref, atol=1e-12)
    # noisy row 0 sees only its own noisy key
    assert torch.allclose(o[..., 0, :], v[..., 0, :], atol=1e-12)


def test_lse_is_logsumexp():
    n, bs, d = 16, 4, 8
    q, k = rand(1, 1, 2 * n, d, seed=1), rand(1, 1, 2 * n, d, seed=2)
    mask = train_mask(n, bs)
    lse = masked_lse(q, k, mask, torch.float64)
    s = (q @ k.transpose(-1, -2)) / d ** 0.5
    for i in range(2 * n):
        vals = s[0, 0, i][mask[i]]
        assert abs(float(lse[0, 0, i]) - float(torch.log(torch.exp(vals).sum()))) < 1e-12


def test_gradcheck_fp64():
    n, bs, d = 4, 2, 4
    q, k, v = (rand(1, 1, 2 * n, d, seed=s + 20).requires_grad_(True) for s in range(3))
    mask = train_mask(n, bs)
    assert torch.autograd.gradcheck(lambda a, b, c: eager_attention(a, b, c, mask, torch.float64), (q, k, v))


def test_backward_closed_forms():
    """dV = P^T dO; dS = P o (dP - Delta) with Delta = rowsum(dO o O);
    dQ = scale dS K; dK = scale dS^T Q; rows of dS sum to 0."""
    n, bs, d = 16, 4, 8
    q, k, v, do = (rand(1, 2, 2 * n, d, seed=s + 30) for s in range(4))
    o, dq, dk, dv = bd3_attention_grads(q, k, v, do, bs, logits_dtype=torch.float64)
    mask = train_mask(n, bs)
    scale = 1 / d ** 0.5
    s = torch.where(mask, q @ k.transpose(-1, -2) * scale, -torch.inf)
    p = torch.softmax(s, -1)
    dp = do @ v.transpose(-1, -2)
    delta = (do * o).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    assert torch.allclose(dv, p.transpose(-1, -2) @ do, atol=1e-12)
    assert torch.allclose(dq, scale * ds @ k, atol=1e-12)
    assert torch.allclose(dk, scale * ds.transpose(-1, -2) @ q, atol=1e-12)
    assert torch.allclose(ds.sum(-1), torch.zeros_like(ds.sum(-1)), atol=1e-12)


def test_chunked_equals_unchunked():
    n, bs, d = 16, 4, 8
    q, k, v, do = (rand(2, 3, 2 * n, d, seed=s + 40) for s in range(4))
    a = bd3_attention(q, k, v, bs, logits_dtype=torch.float64)
    b = bd3_attention(q, k, v, bs, chunk=2, logits_dtype=torch.float64)
    assert all(torch.allclose(x, y, atol=1e-12) for x, y in zip(a, b))
    a = bd3_attention_grads(q, k, v, do, bs, logits_dtype=torch.float64)
    b = bd3_attention_grads(q, k, v, do, bs, chunk=4, logits_dtype=torch.float64)
    assert all(torch.allclose(x, y, atol=1e-12) for x, y in zip(a, b))


@pytest.mark.parametrize("n,bs,rows", [(64, 4, 16), (64, 16, 48), (128, 32, 128), (96, 1, 40)])
def test_row_blocked_grads_equal_autograd(n, bs, rows):
    """The row-blocked closed-form oracle (long sequences) gives the dense
    autograd values, in float64, whatever the row block (including blocks
    that straddle the noisy / clean halves and a ragged last block)."""
    d = 16
    q, k, v, do = (rand(1, 1, 2 * n, d, seed=s + 70)[0, 0].double() for s in range(4))
    o, lse, dq, dk, dv = bd3_attention_grads_rows(q, k, v, do, bs, rows=rows)
    ro, rdq, rdk, rdv = bd3_attention_grads(q[None, None], k[None, None], v[None, None], do[None, None], bs,
                                            logits_dtype=torch.float64)
    _, rlse = bd3_attention(q[None, None], k[None, None], v[None, None], bs, logits_dtype=torch.float64)
    for got, ref in ((o, ro), (lse, rlse), (dq, rdq), (dk, rdk), (dv, rdv)):
        assert torch.allclose(got.double(), ref[0, 0].double(), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("n,bs", [(128, 16), (96, 1), (64, 64)])
def test_key_shift_invariance_pins_delta(n, bs):
    """Shifting every key of a slice by one vector c moves each row's scores
    by a constant, so O, dK and dV stay and dQ moves by scale * (sum_j dS_ij) c,
    which is 0 because Delta = rowsum(dO o O) makes every row of dS sum to 0.
    The oracle (float64) keeps all four; with Delta planted wrong in the
    oracle (zero or doubled) dQ moves by a large fraction of itself, so the
    GPU property test over every slice (tests/test_gpu_train.py) detects a
    wrong Delta without the oracle."""
    from _gpu_util import key_shift_inputs
    q, k, v, do, c = (t[0, 0].double() for t in key_shift_inputs(1, 1, n, seed=n + bs))
    base = bd3_attention_grads_rows(q, k, v, do, bs, rows=64)
    moved = bd3_attention_grads_rows(q, k + c, v, do, bs, rows=64)
    scale = 1.0 / q.shape[-1] ** 0.5
    rel = lambda a, b: float((a - b).norm() / b.norm())
    assert torch.allclose(moved[1] - base[1], (q @ c[0]) * scale, atol=1e-9)  # lse moves by scale * q.c
    for i in (0, 2, 3, 4):  # O, dQ, dK, dV
        assert rel(moved[i], base[i]) < 1e-9
    for factor in (0.0, 2.0):
        planted = bd3_attention_grads_rows(q, k, v, do, bs, rows=64, delta_factor=factor)
        planted_moved = bd3_attention_grads_rows(q, k + c, v, do, bs, rows=64, delta_factor=factor)
        assert rel(planted_moved[2], planted[2]) > 0.1


def test_cached_decode_step_is_unmasked_sdpa():
    q = rand(2, 3, 16, 8, seed=50)
    k, v = rand(2, 3, 160, 8, seed=51), rand(2, 3, 160, 8, seed=52)
    assert torch.allclose(decode_attention(q, k, v, 16, torch.float64), F.scaled_dot_product_attention(q, k, v),
                          atol=1e-12)


def test_decode_prefill_is_block_causal_sdpa():
    L, bs = 48, 8
    q, k, v = (rand(1, 2, L, 8, seed=s + 60) for s in range(3))
    pos = torch.arange(L)
    mask = (pos[None, :] // bs) <= (pos[:, None] // bs)
    assert torch.allclose(decode_attention(q, k, v, bs, torch.float64),
                          F.scaled_dot_product_attention(q, k, v, attn_mask=mask), atol=1e-12)


@pytest.mark.parametrize("bounds", [[(0, 100)], [(0, 37), (37, 100)], [(0, 16), (16, 64), (64, 99), (99, 100)]])
def test_split_merge_equals_full(bounds):
    q = rand(2, 2, 12, 8, seed=70, dtype=torch.float32)
    k, v = rand(2, 2, 100, 8, seed=71, dtype=torch.float32), rand(2, 2, 100, 8, seed=72, dtype=torch.float32)
    parts, lses = split_partials(q, k, v, 4, bounds)
    assert torch.allclose(split_merge(parts, lses), decode_attention(q, k, v, 4), atol=1e-5)


def test_useful_flops_config1():
    """91.604 GFLOP fwd+bwd at B=8, L=1024, H=12, d=64, bs=16 (3.5 x forward)."""
    fwd = useful_flops_fwd(8, 12, 1024, 16)
    assert fwd == 26_172_456_960
    assert abs(3.5 * fwd / 1e9 - 91.604) < 1e-3
