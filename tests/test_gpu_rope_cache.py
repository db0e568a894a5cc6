"""GPU parity of the fused QKV split + RoPE + cache placement (bd3_qkv_rope),
the cache copy (bd3_kv_write) and the preallocated KVCache against the CPU
restatement of the reference (oracle/rope.py): bit-exact, including strided
inputs and outputs, explicit positions, and a sampler-like sequence of
uncommitted denoising steps and commits that grows the cache."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kernels._native import check, lib, ptr, stream_of, strides
from kernels.kv_cache import KVCache, attention_inputs, rope_tables
from kernels.BlockSparseDecodeAttention import block_sparse_decode_attention
from oracle import rope as orc

D = 64


def bits_to_dev(b: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(dev)


def dev_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rand_qkv(B, S, H, seed, scale=2.0):
    x = np.random.default_rng(seed).standard_normal((B, S, 3 * H * D)).astype(np.float32) * scale
    return orc.bf16_bits(x)


@pytest.fixture(scope="module")
def tables():
    return orc.rope_tables(D, 4096)


def dev_tables(tables, dev):
    sin, cos = tables
    return torch.from_numpy(sin).to(dev), torch.from_numpy(cos).to(dev)


@pytest.mark.gpu
def test_rope_tables_match_oracle(cuda, tables):
    sin, cos = rope_tables(D, 4096)
    assert np.array_equal(sin.numpy(), tables[0]) and np.array_equal(cos.numpy(), tables[1])


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,H,pos", [(1, 1, 1, None), (2, 16, 12, 5), (8, 32, 12, "explicit"),
                                       (2, 300, 4, None), (1, 2048, 12, None), (3, 7, 2, "explicit")])
@pytest.mark.parametrize("layout", ["contiguous", "cache_slot"])
def test_qkv_rope_matches_oracle(cuda, tables, B, S, H, pos, layout):
    print(f"qkv_rope B={B} S={S} H={H} pos={pos} layout={layout}", flush=True)
    sin_d, cos_d = dev_tables(tables, cuda)
    x = rand_qkv(B, S, H, seed=B * 1000 + S)
    if pos == "explicit":
        positions = np.random.default_rng(S).integers(0, 4096, S)
        pos_arg = torch.from_numpy(positions).to(cuda)
    elif pos is None:
        positions, pos_arg = np.arange(S), None
    else:
        positions, pos_arg = np.arange(pos, pos + S), pos
    qw, kw, vw = orc.split_qkv(x, H)
    qw, kw = orc.rope_bf16(qw, positions, *tables), orc.rope_bf16(kw, positions, *tables)

    qkv = bits_to_dev(x, cuda)
    q = torch.empty((B, H, S, D), device=cuda, dtype=torch.bfloat16)
    if layout == "contiguous":
        k, v = torch.empty_like(q), torch.empty_like(q)
    else:  # the slot [40, 40 + S) of a (B, H, S + 56, D) cache, surroundings poisoned
        kb = torch.full((B, H, S + 56, D), float("nan"), device=cuda, dtype=torch.bfloat16)
        vb = torch.full_like(kb, float("nan"))
        k, v = kb[:, :, 40:40 + S], vb[:, :, 40:40 + S]
    pos_ptr, pos0 = (ptr(pos_arg), 0) if isinstance(pos_arg, torch.Tensor) else (None, pos_arg or 0)
    xs = (ctypes.c_int64 * 2)(qkv.stride(0), qkv.stride(1))
    check(lib().bd3_qkv_rope(ptr(qkv), xs, B, S, H, D, pos_ptr, pos0, ptr(sin_d), ptr(cos_d), 4096,
                             ptr(q), ptr(k), ptr(v), strides(q, k, v), stream_of(qkv)))
    torch.cuda.synchronize()
    for name, got, want in (("q", q, qw), ("k", k, kw), ("v", v, vw)):
        assert np.array_equal(dev_bits(got), want), name
    if layout == "cache_slot":
        assert torch.isnan(kb[:, :, :40].float()).all() and torch.isnan(kb[:, :, 40 + S:].float()).all()
        assert torch.isnan(vb[:, :, :40].float()).all() and torch.isnan(vb[:, :, 40 + S:].float()).all()


@pytest.mark.gpu
def test_qkv_rope_strided_projection(cuda, tables):
    """The projection read in place from a wider buffer (row stride > width)."""
    B, S, H = 2, 48, 12
    sin_d, cos_d = dev_tables(tables, cuda)
    x = rand_qkv(B, S, H, seed=11)
    wide = torch.zeros((B, S, 3 * H * D + 64), device=cuda, dtype=torch.bfloat16)
    wide[:, :, :3 * H * D] = bits_to_dev(x, cuda)
    q, k_all, v_all = attention_inputs(wide[:, :, :3 * H * D], H, sin_d, cos_d, positions=100)
    qw, kw, vw = orc.attention_inputs(x, H, *tables, positions=np.arange(100, 100 + S))
    for got, want in ((q, qw), (k_all, kw), (v_all, vw)):
        assert np.array_equal(dev_bits(got), want)


@pytest.mark.gpu
def test_kv_write_matches_copy(cuda):
    B, H, S = 2, 12, 40
    k = torch.randn((B, H, S, D), device=cuda).to(torch.bfloat16)
    v = torch.randn((B, H, S, D), device=cuda).to(torch.bfloat16)
    kb = torch.zeros((B, H, 3 * S, D), device=cuda, dtype=torch.bfloat16)
    vb = torch.zeros_like(kb)
    kd, vd = kb[:, :, S:2 * S], vb[:, :, S:2 * S]
    check(lib().bd3_kv_write(ptr(k), ptr(v), ptr(kd), ptr(vd), B, H, S, D, strides(k, v, kd, vd),
                             stream_of(k)))
    torch.cuda.synchronize()
    assert torch.equal(kd, k) and torch.equal(vd, v)
    assert not kb[:, :, :S].any() and not kb[:, :, 2 * S:].any()


@pytest.mark.gpu
@pytest.mark.parametrize("capacity", [None, 4096])
def test_cache_sampler_sequence(cuda, tables, capacity):
    """Blocks of 16 tokens, 3 uncommitted denoising steps then a commit per
    block, 2 layers, 20 blocks (grows past the initial 256-token buffer):
    every (q, k_all, v_all) equals the reference-semantics oracle bit for bit,
    and decode attention over the cache views equals decode over
    concatenated copies."""
    B, H, bs, n_layers = 2, 12, 16, 2
    sin_d, cos_d = dev_tables(tables, cuda)
    cache, ref = KVCache.empty(n_layers, capacity), orc.RefKVCache(n_layers)
    seed = 0
    for blk in range(20):
        start = blk * bs
        for step in range(4):
            store = step == 3
            for layer in range(n_layers):
                seed += 1
                x = rand_qkv(B, bs, H, seed)
                pos = torch.arange(start, start + bs, device=cuda) if layer == 0 else start
                q, k_all, v_all = attention_inputs(bits_to_dev(x, cuda), H, sin_d, cos_d, pos,
                                                   cache, layer, store)
                qw, kw, vw = orc.attention_inputs(x, H, *tables, np.arange(start, start + bs), ref,
                                                  layer, store)
                assert k_all.shape == (B, H, start + bs, D)
                for name, got, want in (("q", q, qw), ("k_all", k_all, kw), ("v_all", v_all, vw)):
                    assert np.array_equal(dev_bits(got), want), (blk, step, layer, name)
                if blk in (0, 19) and layer == 1 and step == 0:
                    o_view = block_sparse_decode_attention(q, k_all, v_all, bs)
                    o_copy = block_sparse_decode_attention(q, k_all.contiguous(), v_all.contiguous(), bs)
                    assert torch.equal(o_view, o_copy)
        assert cache.length == ref.length == start + bs
    for layer in range(n_layers):
        kc, vc = cache.get(layer)
        assert np.array_equal(dev_bits(kc), ref.get(layer)[0])
        assert np.array_equal(dev_bits(vc), ref.get(layer)[1])


@pytest.mark.gpu
def test_cache_append_api(cuda):
    """KVCache.append / get / length against the reference semantics."""
    B, H = 1, 3
    cache, ref = KVCache.empty(2), orc.RefKVCache(2)
    assert cache.length == 0 and cache.get(1) == (None, None)
    rng = np.random.default_rng(3)
    for n in (5, 16, 300, 1):
        for layer in range(2):
            kb = orc.bf16_bits(rng.standard_normal((B, H, n, D)).astype(np.float32))
            vb = orc.bf16_bits(rng.standard_normal((B, H, n, D)).astype(np.float32))
            cache.append(layer, bits_to_dev(kb, cuda), bits_to_dev(vb, cuda))
            ref.append(layer, kb, vb)
        assert cache.length == ref.length
        for layer in range(2):
            kc, vc = cache.get(layer)
            assert np.array_equal(dev_bits(kc), ref.get(layer)[0])
            assert np.array_equal(dev_bits(vc), ref.get(layer)[1])


@pytest.mark.gpu
def test_qkv_rope_extreme_values(cuda, tables):
    """Subnormal, huge, infinite and NaN inputs: the kernel's roundings match
    the oracle's (and so torch's) bit for bit, including overflow to inf and
    the canonical NaN."""
    B, S, H = 1, 64, 4
    rng = np.random.default_rng(21)
    mags = np.array([1e-41, 1e-39, 3e-38, 1.0, 2.5e38, 3.3e38], dtype=np.float32)
    x = (rng.choice(mags, (B, S, 3 * H * D)) * rng.choice([-1.0, 1.0], (B, S, 3 * H * D))).astype(np.float32)
    x.reshape(-1)[rng.integers(0, x.size, 40)] = np.inf
    x.reshape(-1)[rng.integers(0, x.size, 40)] = -np.inf
    x.reshape(-1)[rng.integers(0, x.size, 40)] = np.nan
    xb = orc.bf16_bits(x)
    sin_d, cos_d = dev_tables(tables, cuda)
    q, k, v = attention_inputs(bits_to_dev(xb, cuda), H, sin_d, cos_d, positions=1000)
    qw, kw, vw = orc.attention_inputs(xb, H, *tables, positions=np.arange(1000, 1000 + S))
    for name, got, want in (("q", q, qw), ("k", k, kw), ("v", v, vw)):
        assert np.array_equal(dev_bits(got), want), name
