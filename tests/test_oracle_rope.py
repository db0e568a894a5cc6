"""Pins of oracle/rope.py (CPU): the bf16 rounding against torch's own
conversion, the RoPE tables against the closed form, the rotation against
complex multiplication in float64 (pairing, direction and frequency ladder),
its bf16 op sequence against torch's bf16 tensor arithmetic, the head split
against an index encoding, and the cache against the reference semantics
it restates."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.rope import (RefKVCache, attention_inputs, bf16_bits, bf16_to_f32, rope_bf16,
                         rope_tables, split_qkv)


def torch_bits(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    # The concatenation is float64 (torch's float64 -> bf16 path, which
    # canonicalises NaN to 0x7fc0 as its GPU conversion does); widening the
    # signalling-NaN payloads below to float64 raises numpy's invalid flag.
    with np.errstate(invalid="ignore"):
        x = np.concatenate([
            rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100_000),
            # exact ties: bf16 value + half an ulp, both parities of the kept bit
            (np.arange(1, 4097, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
            (np.arange(1, 4097, dtype=np.uint32) << 16 | 0x7FFF).view(np.float32),
            np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38, np.nan, -np.nan],
                     dtype=np.float32),
            np.array([0x7F800001, 0xFFC12345, 0x7FBFFFFF], dtype=np.uint32).view(np.float32),  # NaN payloads
        ])
    want = torch_bits(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(bf16_bits(x), want)


def test_tables_closed_form():
    d, L, theta = 64, 300, 10000.0
    sin, cos = rope_tables(d, L, theta)
    assert sin.shape == cos.shape == (L, d // 2) and sin.dtype == np.float32
    for p in (0, 1, 7, 123, 299):
        for k in (0, 1, 15, 31):
            ang = p * theta ** (-(2 * k) / d)
            assert sin[p, k] == np.float32(math.sin(ang))
            assert cos[p, k] == np.float32(math.cos(ang))
    assert (sin[0] == 0).all() and (cos[0] == 1).all()


def _rand_bf16(shape, seed, scale=1.0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * scale
    return bf16_bits(x)


def test_rope_against_complex_rotation():
    """Pair (k, k + d/2) as the complex number x_k + i x_{k+d/2}, rotated by
    p * theta^(-2k/d): the bf16 result is within the error of its three
    roundings (plus the table rounding) of the exact rotation."""
    d, S = 64, 200
    sin, cos = rope_tables(d, 4096)
    x = _rand_bf16((3, S, d), 1)
    pos = np.random.default_rng(2).integers(0, 4096, S)
    got = bf16_to_f32(rope_bf16(x, pos, sin, cos)).astype(np.float64)
    xf = bf16_to_f32(x).astype(np.float64)
    z = xf[..., :32] + 1j * xf[..., 32:]
    ang = np.outer(pos, 10000.0 ** (-np.arange(0, d, 2) / d))
    w = z * np.exp(1j * ang)
    exact = np.concatenate([w.real, w.imag], axis=-1)
    mag = np.abs(np.concatenate([z, z], axis=-1))
    err = np.abs(got - exact)
    assert (err <= 5 * 2.0 ** -8 * mag + 1e-30).all(), float((err / (mag + 1e-30)).max())
    # a plausible slip (opposite rotation, or interleaved pairs) is far outside the bound
    wrong = z * np.exp(-1j * ang)
    assert np.abs(got - np.concatenate([wrong.real, wrong.imag], -1)).max() > 0.5


def test_rope_position_zero_is_identity():
    sin, cos = rope_tables(64, 8)
    x = _rand_bf16((2, 5, 64), 3)
    assert np.array_equal(rope_bf16(x, np.zeros(5, dtype=np.int64), sin, cos), x)


def test_rope_relative_positions():
    """<R(p) q, R(p') k> depends on p - p' only (float64 tables)."""
    sin, cos = rope_tables(64, 512)
    rng = np.random.default_rng(4)
    q, k = rng.standard_normal(64), rng.standard_normal(64)

    def rot(x, p):
        ang = p * 10000.0 ** (-np.arange(0, 64, 2) / 64)
        c, s = np.cos(ang), np.sin(ang)
        return np.concatenate([x[:32] * c - x[32:] * s, x[:32] * s + x[32:] * c])

    base = rot(q, 10) @ rot(k, 3)
    for shift in (1, 50, 400):
        assert abs(rot(q, 10 + shift) @ rot(k, 3 + shift) - base) < 1e-9


def test_rope_matches_torch_bf16_ops():
    """The oracle's rounding sequence equals torch's bf16 tensor arithmetic
    on the reference's expression (model/modules.py:233-240)."""
    sin, cos = rope_tables(64, 2048)
    x = _rand_bf16((2, 3, 77, 64), 5, scale=3.0)
    pos = np.random.default_rng(6).integers(0, 2048, 77)
    xt = from_bits(x)
    s = torch.from_numpy(sin)[torch.from_numpy(pos)].to(torch.bfloat16)
    c = torch.from_numpy(cos)[torch.from_numpy(pos)].to(torch.bfloat16)
    x1, x2 = xt.chunk(2, dim=-1)
    want = torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)
    assert np.array_equal(rope_bf16(x, pos, sin, cos), torch_bits(want))


def test_split_qkv_index_encoding():
    B, S, H, d = 2, 5, 3, 64
    b, s, t, h, j = np.meshgrid(np.arange(B), np.arange(S), np.arange(3), np.arange(H), np.arange(d),
                                indexing="ij")
    code = (((b * S + s) * 3 + t) * H + h) * d + j
    qkv = code.reshape(B, S, 3 * H * d).astype(np.uint32)
    q, k, v = split_qkv(qkv, H)
    for ti, part in enumerate((q, k, v)):
        assert part.shape == (B, H, S, d)
        for bb, hh, ss, jj in [(0, 0, 0, 0), (1, 2, 4, 63), (0, 1, 3, 17)]:
            assert part[bb, hh, ss, jj] == (((bb * S + ss) * 3 + ti) * H + hh) * d + jj


def test_cache_semantics():
    sin, cos = rope_tables(64, 256)
    H = 2
    cache = RefKVCache(2)
    assert cache.length == 0 and cache.get(0) == (None, None)
    qkv0 = _rand_bf16((1, 16, 3 * H * 64), 7)
    q, k_all, v_all = attention_inputs(qkv0, H, sin, cos, None, cache, 0, store=True)
    assert k_all.shape == (1, H, 16, 64) and cache.length == 16
    qkv1 = _rand_bf16((1, 16, 3 * H * 64), 8)
    _, k_all, v_all = attention_inputs(qkv1, H, sin, cos, np.arange(16, 32), cache, 0, store=False)
    assert k_all.shape == (1, H, 32, 64) and cache.length == 16
    assert np.array_equal(k_all[:, :, :16], cache.get(0)[0])
    # the uncached call over the whole prefix produces the same keys (prefill == commit)
    both = np.concatenate([qkv0, qkv1], axis=1)
    _, k_full, v_full = attention_inputs(both, H, sin, cos)
    assert np.array_equal(k_full, k_all) and np.array_equal(v_full, v_all)
