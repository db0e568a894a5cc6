"""The Python mirror keeps the reference's kernel-module interface
(kernels/BlockSparseFlashAttention.py, kernels/BlockSparseDecodeAttention.py,
kernels/SplitKVDecodeAttention.py, bench/attention.py) and its error
behaviour; checked without a GPU."""
import inspect
import types

import pytest
import torch

from kernels import backends
from kernels.BlockSparseDecodeAttention import _last_stride_1, block_sparse_decode_attention
from kernels.BlockSparseFlashAttention import BlockSparseFlashAttention
from kernels.SplitKVDecodeAttention import SPLIT_N, split_kv_decode_attention


def params(fn):
    return list(inspect.signature(fn).parameters)


def test_signatures():
    assert params(BlockSparseFlashAttention.forward) == ["ctx", "q", "k", "v", "block_size"]
    assert params(BlockSparseFlashAttention.backward) == ["ctx", "dO"]
    assert params(block_sparse_decode_attention) == ["q", "k", "v", "block_size"]
    assert params(split_kv_decode_attention)[:4] == ["q", "k", "v", "block_size"]
    assert inspect.signature(split_kv_decode_attention).parameters["n_splits"].default is None
    assert SPLIT_N == 256
    for name in ("FWD_BLOCK_M", "FWD_BLOCK_N", "BWD_DQ_BLOCK_M", "BWD_DKDV_BLOCK_KV", "BWD_DKDV_BLOCK_Q"):
        assert isinstance(getattr(BlockSparseFlashAttention, name), int)


def test_cpu_tensors_raise_assertion():
    q = torch.zeros(1, 1, 256, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="CUDA"):
        BlockSparseFlashAttention.apply(q, q, q, 16)


def test_odd_sequence_raises():
    q = torch.zeros(1, 1, 255, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        BlockSparseFlashAttention.apply(q, q, q, 16)


def test_decode_q_longer_than_kv_raises():
    q = torch.zeros(1, 1, 17, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 16, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="last q_len"):
        block_sparse_decode_attention(q, k, k, 16)
    with pytest.raises(AssertionError, match="last q_len"):
        split_kv_decode_attention(q, k, k, 16)


def test_last_stride_1():
    x = torch.zeros(2, 3, 4, 8).transpose(-1, -2)
    assert _last_stride_1(x).stride(-1) == 1
    y = torch.zeros(2, 3, 4, 8)
    assert _last_stride_1(y) is y


def test_registry_and_install():
    assert set(backends.BLOCK_SIZE_BACKENDS) == {"bsfa", "bsdfa", "split_kv"}
    for name in backends.BLOCK_SIZE_BACKENDS:
        assert params(backends.BACKENDS[name]) == ["q", "k", "v", "mask", "block_size"]
    model_module = types.ModuleType("fake_modules")
    model_module.scaled_dot_product_attention = lambda q, k, v, mask=None: None
    with pytest.raises(AssertionError, match="block_size"):
        backends.install_attention("bsfa", module=model_module)
    fn = backends.install_attention("split_kv", block_size=16, module=model_module)
    assert model_module.scaled_dot_product_attention is fn
    assert fn.keywords == {"block_size": 16}
    ranged = backends.install_attention("bsdfa", nvtx=True, block_size=16, module=model_module)
    assert model_module.scaled_dot_product_attention is ranged
