"""Rotary embedding, fused-QKV head split and KV cache of one BD3-LM attention
layer, on the CPU. Test infrastructure only (see oracle/__init__.py).

Restates, with numpy (bf16 values carried as uint16 bit patterns):
* the RoPE tables (model/modules.py:190-210): angles p * theta^(-2k/d) in
  float64 for pair k = 0 .. d/2-1, sin and cos cast to float32;
* RoPE.forward (model/modules.py:212-240): the table rows of the positions
  cast to x's dtype (bf16), rotate-half pairing of coordinate k with k + d/2,
  out1 = x1*cos - x2*sin and out2 = x1*sin + x2*cos, where every product,
  the difference and the sum is a separate bf16 tensor op (fp32 arithmetic,
  result rounded to nearest even);
* the head split "... seq (three n_heads d_k) -> three ... n_heads seq d_k"
  (model/modules.py:395-403);
* the cache: KVCache (model/kv_cache.py:8-55) and k_all = cat(cache, k),
  v_all = cat(cache, v), then append when store (model/modules.py:409-417).
"""
from __future__ import annotations

import numpy as np


def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even; every NaN becomes
    the canonical quiet NaN 0x7fc0 (torch's conversion)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, np.uint32(0x7FC0), r)
    return r.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _rnd(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 and back (one bf16 tensor op's output)."""
    return bf16_to_f32(bf16_bits(x))


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0) -> tuple[np.ndarray, np.ndarray]:
    """(sin, cos), each float32 (max_seq_len, head_dim/2) (model/modules.py:190-210)."""
    assert head_dim % 2 == 0
    pos = np.arange(max_seq_len, dtype=np.float64)
    inv_freq = theta ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    angles = np.outer(pos, inv_freq)
    return np.sin(angles).astype(np.float32), np.cos(angles).astype(np.float32)


def rope_bf16(x_bits: np.ndarray, positions, sin: np.ndarray, cos: np.ndarray) -> np.ndarray:
    """RoPE.forward on bf16 x (..., seq, d) (model/modules.py:212-240); returns bf16 bits."""
    positions = np.asarray(positions)
    s = _rnd(sin[positions])  # (seq, d/2): .to(x.dtype)
    c = _rnd(cos[positions])
    x = bf16_to_f32(x_bits)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    # bf16 inputs near the format's maximum overflow to +-inf (and inf - inf
    # gives NaN) exactly as torch's bf16 ops do; that is the expected result.
    with np.errstate(over="ignore", invalid="ignore"):
        out1 = _rnd(_rnd(x1 * c) - _rnd(x2 * s))
        out2 = _rnd(_rnd(x1 * s) + _rnd(x2 * c))
    return bf16_bits(np.concatenate([out1, out2], axis=-1))


def split_qkv(qkv_bits: np.ndarray, n_heads: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(batch, seq, 3*n_heads*d) -> q, k, v each (batch, n_heads, seq, d)
    (model/modules.py:398-403)."""
    B, S, W = qkv_bits.shape
    d = W // (3 * n_heads)
    t = qkv_bits.reshape(B, S, 3, n_heads, d).transpose(2, 0, 3, 1, 4)
    return tuple(np.ascontiguousarray(t[i]) for i in range(3))


class RefKVCache:
    """KVCache with the reference's semantics (model/kv_cache.py:8-55):
    one (k, v) slot per layer, None until the first append, grown by
    concatenation along the sequence axis."""

    def __init__(self, n_layers: int):
        self.k: list[np.ndarray | None] = [None] * n_layers
        self.v: list[np.ndarray | None] = [None] * n_layers

    @property
    def length(self) -> int:
        return 0 if self.k[0] is None else self.k[0].shape[-2]

    def get(self, layer_idx: int):
        return self.k[layer_idx], self.v[layer_idx]

    def append(self, layer_idx: int, k: np.ndarray, v: np.ndarray) -> None:
        sk, sv = self.get(layer_idx)
        if sk is None or sv is None:
            self.k[layer_idx], self.v[layer_idx] = k, v
        else:
            self.k[layer_idx] = np.concatenate([sk, k], axis=-2)
            self.v[layer_idx] = np.concatenate([sv, v], axis=-2)


def attention_inputs(qkv_bits: np.ndarray, n_heads: int, sin: np.ndarray, cos: np.ndarray,
                     positions=None, kv_cache: RefKVCache | None = None, layer_idx: int = 0,
                     store: bool = False):
    """(q, k_all, v_all) as BidirectionalMultiHeadAttention.forward builds
    them before attention (model/modules.py:395-417), bf16 bits."""
    q, k, v = split_qkv(qkv_bits, n_heads)
    if positions is None:
        positions = np.arange(q.shape[-2])
    q = rope_bf16(q, positions, sin, cos)
    k = rope_bf16(k, positions, sin, cos)
    k_all, v_all = k, v
    if kv_cache is not None:
        kc, vc = kv_cache.get(layer_idx)
        if kc is not None and vc is not None:
            k_all = np.concatenate([kc, k], axis=-2)
            v_all = np.concatenate([vc, v], axis=-2)
    if store and kv_cache is not None:
        kv_cache.append(layer_idx, k, v)
    return q, k_all, v_all
