"""BD3-LM masks, restated with numpy (integer arithmetic, bit-exact).
Test infrastructure only (see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np


def block_diff_mask(n: int, block_size: int) -> np.ndarray:
    """(2n, 2n) bool training mask over cat(x_t, x_0).

    Follows model/bd3lm.py:34-52: query/key index < n is noisy, block id is
    (index % n) // block_size;
        noisy q -> noisy k, same block            (block diagonal, :48)
        noisy q -> clean k, strictly earlier block (offset block-causal, :49)
        clean q -> clean k, same or earlier block  (block-causal, :50)
    """
    idx = np.arange(2 * n)
    q = idx[:, None]
    k = idx[None, :]
    q_clean, k_clean = q >= n, k >= n
    q_block = (q % n) // block_size
    k_block = (k % n) // block_size
    block_diagonal = ~q_clean & ~k_clean & (q_block == k_block)
    offset_block_causal = ~q_clean & k_clean & (k_block < q_block)
    block_causal = q_clean & k_clean & (k_block <= q_block)
    return block_diagonal | offset_block_causal | block_causal


def decode_mask(q_len: int, kv_len: int, block_size: int) -> np.ndarray:
    """(q_len, kv_len) bool mask of the decode kernels: queries are the last
    q_len of kv_len positions, block-causal over positions.

    Follows kernels/BlockSparseDecodeAttention.py:84-85 (q_block of row i is
    (kv_len - q_len + i) // block_size) and _decode_tiles :23-26
    (q_block >= kv_idx // block_size and kv_idx < kv_len). It equals the
    clean-clean slice the uncached sampler uses, model/bd3lm.py:168.
    """
    rows = (kv_len - q_len + np.arange(q_len))[:, None]
    keys = np.arange(kv_len)[None, :]
    return (rows // block_size) >= (keys // block_size)


def pair_count(n: int, block_size: int) -> int:
    """Live pairs of block_diff_mask(n, block_size) when n % block_size == 0:
    n^2 + n * block_size (noisy rows see bs own + bs*b clean keys, clean rows
    bs*(b+1); summing over blocks gives n^2 + n*bs)."""
    assert n % block_size == 0
    return n * n + n * block_size


def live_tile_fraction(mask: np.ndarray, tile_m: int, tile_n: int) -> float:
    """Fraction of (tile_m x tile_n) tiles of `mask` holding any live pair."""
    R, C = mask.shape
    t = mask.reshape(R // tile_m, tile_m, C // tile_n, tile_n).any(axis=(1, 3))
    return float(t.mean())
