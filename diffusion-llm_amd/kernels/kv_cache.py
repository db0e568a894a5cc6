"""KV cache and fused attention inputs for BD3-LM sampling, on MI355X.

`KVCache` is a drop-in for the reference's model/kv_cache.py:8-55 (same
`empty(n_layers)`, `length`, `get(layer_idx)`, `append(layer_idx, k, v)`),
but each layer's keys and values live in one preallocated
(batch, heads, capacity, head_dim) buffer: `append` writes the new tokens
into the slot [length, length + new) instead of reallocating with torch.cat,
and `get` returns views of the committed prefix, which the decode kernels
read in place. The buffer doubles when it fills (one copy, amortised).

`attention_inputs` produces (q, k_all, v_all) exactly as
BidirectionalMultiHeadAttention.forward does before it calls attention
(model/modules.py:395-417): head split of the fused projection, RoPE on q and
k, concatenation with the cached prefix, and the append when `store`. One
bd3_qkv_rope launch writes q and places k / v straight into the cache slot
after the committed prefix, so k_all / v_all are views of the cache and the
per-step copy of the whole cache disappears. Results are bit-identical to
the reference's eager bf16 path.

With a cache, k_all / v_all alias the layer's buffer: the block's slot is
overwritten by the next uncommitted call for that layer (the sampler
consumes them immediately, as the reference does).
"""
from __future__ import annotations

import ctypes
import math

import torch
from torch import Tensor

from kernels._native import as_kernel_input, check, lib, ptr, stream_of, strides

_MIN_CAPACITY = 256


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0,
                device: torch.device | None = None) -> tuple[Tensor, Tensor]:
    """(sin_table, cos_table), float32 (max_seq_len, head_dim / 2): the RoPE
    module's buffers (model/modules.py:190-210), angles p * theta^(-2k/d)
    formed in float64."""
    assert head_dim % 2 == 0, f"head_dim must be even, got {head_dim}"
    pos = torch.arange(max_seq_len, dtype=torch.float64, device=device)
    inv_freq = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64, device=device) / head_dim)
    angles = torch.outer(pos, inv_freq)
    return torch.sin(angles).float(), torch.cos(angles).float()


def _copy_kv(k: Tensor, v: Tensor, k_dst: Tensor, v_dst: Tensor) -> None:
    B, H, S, D = k.shape
    check(lib().bd3_kv_write(ptr(k), ptr(v), ptr(k_dst), ptr(v_dst), B, H, S, D,
                             strides(k, v, k_dst, v_dst), stream_of(k)))


class KVCache:
    """Per-layer post-RoPE keys / values of committed blocks
    (reference: model/kv_cache.py:8-55), in preallocated buffers."""

    def __init__(self, n_layers: int, capacity: int | None = None):
        self._k: list[Tensor | None] = [None] * n_layers
        self._v: list[Tensor | None] = [None] * n_layers
        self._len = [0] * n_layers
        self._capacity = capacity

    @classmethod
    def empty(cls, n_layers: int, capacity: int | None = None) -> "KVCache":
        """A cache with no committed tokens, one slot per layer. `capacity`
        (tokens) sizes the buffers up front; otherwise they start at the
        first append's need and double as they fill."""
        return cls(n_layers, capacity)

    @property
    def length(self) -> int:
        """Number of committed tokens (of layer 0, as the reference)."""
        return self._len[0]

    def get(self, layer_idx: int) -> tuple[Tensor | None, Tensor | None]:
        """Views (batch, heads, length, head_dim) of the committed keys and
        values of one layer, or (None, None) if nothing is committed."""
        n = self._len[layer_idx]
        if n == 0:
            return None, None
        return self._k[layer_idx][:, :, :n], self._v[layer_idx][:, :, :n]

    def _reserve(self, layer_idx: int, like: Tensor, need: int) -> None:
        """Make layer_idx's buffers hold `need` tokens of like's
        (batch, heads, *, head_dim) shape and dtype."""
        B, H, _, D = like.shape
        buf = self._k[layer_idx]
        if buf is not None:
            assert buf.shape[0] == B and buf.shape[1] == H and buf.shape[3] == D, \
                "cached and new keys differ in batch, heads or head_dim"
            assert buf.dtype == like.dtype and buf.device == like.device, "cache dtype / device mismatch"
            if buf.shape[2] >= need:
                return
        cap = max(need, self._capacity or 0, _MIN_CAPACITY, 2 * (buf.shape[2] if buf is not None else 0))
        cap = 8 * math.ceil(cap / 8)
        k_new = torch.empty((B, H, cap, D), device=like.device, dtype=like.dtype)
        v_new = torch.empty_like(k_new)
        n = self._len[layer_idx]
        if n > 0:
            _copy_kv(self._k[layer_idx][:, :, :n], self._v[layer_idx][:, :, :n],
                     k_new[:, :, :n], v_new[:, :, :n])
        self._k[layer_idx], self._v[layer_idx] = k_new, v_new

    def slot(self, layer_idx: int, like: Tensor, new: int) -> tuple[Tensor, Tensor]:
        """Views of the `new` token positions after the committed prefix
        (capacity grown if needed); not committed until `commit`."""
        n = self._len[layer_idx]
        self._reserve(layer_idx, like, n + new)
        return self._k[layer_idx][:, :, n:n + new], self._v[layer_idx][:, :, n:n + new]

    def prefix_and_slot(self, layer_idx: int, new: int) -> tuple[Tensor, Tensor]:
        """Views of the committed prefix plus the slot: (batch, heads, length + new, d)."""
        n = self._len[layer_idx] + new
        return self._k[layer_idx][:, :, :n], self._v[layer_idx][:, :, :n]

    def commit(self, layer_idx: int, new: int) -> None:
        self._len[layer_idx] += new

    def append(self, layer_idx: int, k: Tensor, v: Tensor) -> None:
        """Append one layer's post-RoPE keys / values of newly committed
        tokens (reference :42-55): one strided copy into the slot."""
        assert k.shape == v.shape and k.dim() == 4, "k and v must be (batch, heads, new, head_dim)"
        assert k.dtype == torch.bfloat16 and k.is_cuda, "bf16 CUDA tensors only"
        new = k.shape[2]
        ks, vs = self.slot(layer_idx, k, new)
        _copy_kv(as_kernel_input(k), as_kernel_input(v), ks, vs)
        self.commit(layer_idx, new)


def attention_inputs(
    qkv: Tensor,  # (batch, seq, 3 * n_heads * head_dim): the fused projection's output
    n_heads: int,
    sin_table: Tensor,  # (max_seq_len, head_dim / 2) float32, on qkv's device
    cos_table: Tensor,
    positions: Tensor | int | None = None,
    kv_cache: KVCache | None = None,
    layer_idx: int = 0,
    store: bool = False,
) -> tuple[Tensor, Tensor, Tensor]:
    """(q, k_all, v_all), each (batch, n_heads, *, head_dim) bf16, as
    model/modules.py:395-417 builds them. `positions`: None = 0 .. seq-1,
    an int = the first of seq consecutive positions, or an integer tensor
    (seq,) of absolute positions (reference: RoPE.forward, :212-240)."""
    assert not store or kv_cache is not None, "store=True needs a kv_cache to store into"
    assert qkv.dim() == 3 and qkv.is_cuda and qkv.dtype == torch.bfloat16, \
        "qkv must be a (batch, seq, 3 * d_model) bf16 CUDA tensor"
    B, S, W = qkv.shape
    assert W % (3 * n_heads) == 0, "projection width must be 3 * n_heads * head_dim"
    D = W // (3 * n_heads)
    assert D == 64, "head_dim must be 64"
    if not (qkv.stride(-1) == 1 and qkv.data_ptr() % 16 == 0 and qkv.stride(0) % 8 == 0
            and qkv.stride(1) % 8 == 0):
        qkv = qkv.contiguous()
    assert sin_table.dtype == cos_table.dtype == torch.float32 and sin_table.shape == cos_table.shape
    assert sin_table.shape[1] == D // 2, "RoPE tables must be (max_seq_len, head_dim / 2)"
    sin_table, cos_table = sin_table.contiguous(), cos_table.contiguous()
    max_pos = sin_table.shape[0]

    pos_ptr, pos0 = None, 0
    if isinstance(positions, int):
        pos0 = positions
    elif positions is not None:
        assert positions.shape == (S,), "positions must be (seq,)"
        positions = positions.to(device=qkv.device, dtype=torch.int64).contiguous()
        pos_ptr = ptr(positions)

    q = torch.empty((B, n_heads, S, D), device=qkv.device, dtype=qkv.dtype)
    if kv_cache is None:
        k_out = torch.empty_like(q)
        v_out = torch.empty_like(q)
    else:
        k_out, v_out = kv_cache.slot(layer_idx, q, S)
    xstr = (ctypes.c_int64 * 2)(qkv.stride(0), qkv.stride(1))
    check(lib().bd3_qkv_rope(ptr(qkv), xstr, B, S, n_heads, D, pos_ptr, pos0, ptr(sin_table),
                             ptr(cos_table), max_pos, ptr(q), ptr(k_out), ptr(v_out),
                             strides(q, k_out, v_out), stream_of(qkv)))
    if kv_cache is None:
        return q, k_out, v_out
    k_all, v_all = kv_cache.prefix_and_slot(layer_idx, S)
    if store:
        kv_cache.commit(layer_idx, S)
    return q, k_all, v_all
