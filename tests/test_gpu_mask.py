"""The mask the device predicate applies equals block_diff_mask and the
decode slice bit for bit (bd3_mask_dump through the C ABI)."""
import numpy as np
import pytest
import torch

from kernels._native import check, lib, ptr
from oracle.mask import block_diff_mask, decode_mask


@pytest.mark.gpu
@pytest.mark.parametrize("n,bs", [(4, 1), (8, 3), (128, 1), (128, 16), (256, 4), (256, 16),
                                  (256, 64), (256, 256), (320, 7), (1024, 16)])
def test_train_mask_bit_exact(cuda, n, bs):
    out = torch.empty((2 * n, 2 * n), device=cuda, dtype=torch.uint8)
    check(lib().bd3_mask_dump(ptr(out), 0, n, 0, bs, None))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().astype(bool), block_diff_mask(n, bs))


@pytest.mark.gpu
@pytest.mark.parametrize("q_len,kv_len,bs", [(16, 16, 16), (16, 4112, 16), (32, 2048, 32),
                                             (1, 37, 4), (3088, 3088, 16), (100, 300, 7)])
def test_decode_mask_bit_exact(cuda, q_len, kv_len, bs):
    out = torch.empty((q_len, kv_len), device=cuda, dtype=torch.uint8)
    check(lib().bd3_mask_dump(ptr(out), 1, q_len, kv_len, bs, None))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().astype(bool), decode_mask(q_len, kv_len, bs))
