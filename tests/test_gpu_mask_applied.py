"""The masks the attention kernels apply, checked exactly on the GPU.

The device mask dump (test_gpu_mask.py) checks the predicate; these tests
check what each kernel actually does with it (strip tests, per-element key
indices, dead / full / partial classes, split boundaries) by making every
kernel output an exact function of the visible key sets.

With q = 0 every score is 0, so every visible key of a row gets the same
weight (references: model/bd3lm.py:10-52, kernels/BlockSparseDecodeAttention.py:84-88):
  * forward: lse_i = ln(c_i), c_i the row's visible-key count, and
    O_i = mean of the visible V rows. With V_j one-hot on a bucket f(j),
    O_i[d] * c_i is the number of visible keys in bucket d (an integer).
  * dQ stage, fed lse = 0 and O = 0 (so Delta = 0), dO_i = e_0 and V_j all
    ones: P = 1 and dS = 1 on visible pairs, so dQ_i = scale * sum of the
    visible K rows; with K_j one-hot on f(j), dQ_i[d] * 8 is an integer
    count (exact in bf16).
  * dK/dV stage, fed Delta = 0 and -L / scale = 0, K = 0, V_j all ones,
    Q_i one-hot on g(i), dO_i one-hot on h(i): dV_j[d] counts the rows that
    see key j with h(i) = d, dK_j[d] * 8 those with g(i) = d (the transposed
    mask, exact integers).
  * decode: O_i[d] = (visible keys of bucket d) / c_i, compared against the
    exact fractions within one bf16 ulp; one key more or less moves the
    affected entry by at least 1/count of its bucket, several ulps.
Two bucket maps, j mod 64 and (j // 64) mod 64, pin each visible set.
"""
import numpy as np
import pytest
import torch

from _gpu_util import D, splitkv_capi
from kernels._native import check, lib, ptr, stream_of, strides
from oracle.mask import block_diff_mask, decode_mask

SCALE = 1.0 / D ** 0.5
BUCKETS = {"mod64": lambda j: j % 64, "div64": lambda j: (j // 64) % 64}

# (n, block size): MASK16 instances (bs % 16 == 0) and per-element ones.
TRAIN = [(128, 1), (384, 3), (128, 4), (384, 8), (896, 7), (256, 16), (256, 32), (1024, 16), (2048, 16),
         (256, 64), (512, 100), (512, 256), (2048, 256)]


def onehot_rows(n_rows, bucket, scale=1.0):
    """(n_rows, 64) float rows, row j one-hot at bucket(j)."""
    m = np.zeros((n_rows, D), dtype=np.float32)
    m[np.arange(n_rows), bucket(np.arange(n_rows))] = scale
    return m


def histogram(mask: np.ndarray, bucket) -> np.ndarray:
    """(rows, 64) int: visible keys of each row per bucket."""
    # float64 BLAS product of 0/1 matrices: exact for counts < 2^53
    return np.rint(mask.astype(np.float64) @ onehot_rows(mask.shape[1], bucket).astype(np.float64)).astype(np.int64)


def dev(a: np.ndarray, heads: int, device) -> torch.Tensor:
    """(S, 64) -> (1, heads, S, 64) bf16 on the device (the same rows per head)."""
    t = torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    return t.expand(1, heads, *t.shape).contiguous().to(device)


def fwd(q, k, v, bs):
    B, H, S, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), device=q.device, dtype=torch.float32)
    check(lib().bd3_attn_fwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, S // 2, D, bs,
                             strides(q, k, v, o), SCALE, stream_of(q)))
    return o, lse


@pytest.mark.gpu
@pytest.mark.parametrize("n,bs", TRAIN)
def test_forward_applies_mask_exactly(cuda, n, bs):
    print(f"forward mask n={n} bs={bs}", flush=True)
    H, S = 2, 2 * n
    mask = block_diff_mask(n, bs)
    counts = mask.sum(axis=1)
    zeros = dev(np.zeros((S, D), np.float32), H, cuda)
    for name, bucket in BUCKETS.items():
        v = dev(onehot_rows(S, bucket), H, cuda)
        o, lse = fwd(zeros, zeros, v, bs)
        torch.cuda.synchronize()
        lse = lse[0].double().cpu().numpy()
        # the count: ln(c) and ln(c + 1) differ by > 1/(c + 1) >= 1/4097
        np.testing.assert_allclose(lse, np.broadcast_to(np.log(counts), lse.shape), rtol=0, atol=2e-5)
        got = o[0].double().cpu().numpy() * counts[None, :, None]
        hist = histogram(mask, bucket)
        assert np.abs(got - hist[None]).max() < 0.25, f"{name}: visible-key histogram differs"
        assert np.array_equal(np.rint(got), np.broadcast_to(hist, got.shape)), name


@pytest.mark.gpu
@pytest.mark.parametrize("n,bs", [c for c in TRAIN if c[0] % c[1] == 0])
def test_dq_kernel_applies_mask_exactly(cuda, n, bs):
    print(f"dQ mask n={n} bs={bs}", flush=True)
    H, S = 2, 2 * n
    mask = block_diff_mask(n, bs)
    zeros = dev(np.zeros((S, D), np.float32), H, cuda)
    ones = dev(np.ones((S, D), np.float32), H, cuda)
    dout = dev(onehot_rows(S, lambda i: 0 * i), H, cuda)  # e_0 rows
    lse = torch.zeros((1, H, S), device=cuda, dtype=torch.float32)
    for name, bucket in BUCKETS.items():
        k = dev(onehot_rows(S, bucket), H, cuda)
        dq = torch.empty_like(zeros)
        ws = torch.empty((2, 1, H, S), device=cuda, dtype=torch.float32)
        # q = 0: P = exp(0 - lse) = 1 on visible pairs; O = 0: Delta = 0; dP = dO . V = 1
        check(lib().bd3_attn_bwd_dq(ptr(zeros), ptr(k), ptr(ones), ptr(zeros), ptr(dout), ptr(lse), ptr(dq),
                                    ptr(ws), 1, H, n, D, bs, strides(zeros, k, ones, zeros, dout, dq), SCALE,
                                    stream_of(k)))
        torch.cuda.synchronize()
        got = dq[0].double().cpu().numpy() / SCALE
        hist = histogram(mask, bucket)
        assert np.array_equal(got, np.broadcast_to(hist, got.shape).astype(np.float64)), \
            f"{name}: dQ histogram differs (max {np.abs(got - hist[None]).max()})"
        assert float(ws[0].abs().max()) == 0.0  # Delta of O = 0


@pytest.mark.gpu
@pytest.mark.parametrize("entry", ["dkdv_stage", "main_launch"])
@pytest.mark.parametrize("n,bs", [c for c in TRAIN if c[0] % c[1] == 0])
def test_dkdv_kernel_applies_transposed_mask_exactly(cuda, n, bs, entry):
    """dK / dV through the dK/dV stage (bd3_attn_bwd_dkdv: a dK/dV item per
    key tile) and through the main launch (bd3_attn_bwd_main: with a block
    size dividing 32 the noisy key tiles' diagonal blocks come from the dQ
    items of the same rows)."""
    print(f"dK/dV mask n={n} bs={bs} via {entry}", flush=True)
    H, S = 2, 2 * n
    mask = block_diff_mask(n, bs)
    zeros = dev(np.zeros((S, D), np.float32), H, cuda)
    ones = dev(np.ones((S, D), np.float32), H, cuda)
    planes = torch.zeros((2, 1, H, S), device=cuda, dtype=torch.float32)  # Delta = 0, -L / scale = 0
    lse = torch.zeros((1, H, S), device=cuda, dtype=torch.float32)
    for (gname, gmap), (hname, hmap) in ((("mod64", BUCKETS["mod64"]), ("div64", BUCKETS["div64"])),
                                         (("div64", BUCKETS["div64"]), ("mod64", BUCKETS["mod64"]))):
        q = dev(onehot_rows(S, gmap), H, cuda)
        dout = dev(onehot_rows(S, hmap), H, cuda)
        dk, dv = torch.empty_like(zeros), torch.empty_like(zeros)
        if entry == "dkdv_stage":
            check(lib().bd3_attn_bwd_dkdv(ptr(q), ptr(zeros), ptr(ones), ptr(dout), ptr(lse), ptr(planes), ptr(dk),
                                          ptr(dv), 1, H, n, D, bs, strides(q, zeros, ones, dout, dk, dv), SCALE,
                                          stream_of(q)))
        else:
            dq = torch.empty_like(zeros)
            check(lib().bd3_attn_bwd_main(ptr(q), ptr(zeros), ptr(ones), ptr(dout), ptr(lse), ptr(planes), ptr(dq),
                                          ptr(dk), ptr(dv), 1, H, n, D, bs,
                                          strides(q, zeros, ones, dout, dq, dk, dv), SCALE, stream_of(q)))
        torch.cuda.synchronize()
        # key j's column: rows i that see j, per bucket of i
        want_k = histogram(mask.T, gmap).astype(np.float64)
        want_v = histogram(mask.T, hmap).astype(np.float64)
        got_k = dk[0].double().cpu().numpy() / SCALE
        got_v = dv[0].double().cpu().numpy()
        assert np.array_equal(got_v, np.broadcast_to(want_v, got_v.shape)), \
            f"dV ({hname}) differs (max {np.abs(got_v - want_v[None]).max()})"
        assert np.array_equal(got_k, np.broadcast_to(want_k, got_k.shape)), \
            f"dK ({gname}) differs (max {np.abs(got_k - want_k[None]).max()})"


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """One bf16 ulp at |x| (2^-7 relative to the leading power of two)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-30)))
    return np.where(x == 0, 0.0, 2.0 ** (e - 7))


DECODE = [  # (q_len, kv_len, block size, split counts)
    (16, 4112, 16, (1, 4, 8, 16, 17)),
    (16, 3584 + 16, 16, (1, 7)),
    (3, 515, 1, (1, 2, 5)),
    (16, 1000, 7, (1, 3, 16)),
    (16, 640, 100, (1, 2)),
    (32, 2048, 32, (1, 3, 4)),
    (40, 1337, 4, (1, 2, 5)),
    (64, 777, 64, (1, 3)),
    # q_len > 64: the prefill kernel (128-row tiles, splits of whole 64-key
    # tiles; single-split row tiles write O, the others go through partials)
    (256, 2048, 256, (1, 3)),
    (300, 300, 16, (1, 2, 5)),  # q_len == kv_len
    (1000, 1000, 16, (1, 3)),  # row tiles 0-2 in the first split, 3-7 merged
    (100, 777, 7, (1, 2, 4)),  # per-element mask, ragged last key tile
    (65, 2048, 32, (1, 5)),  # the tile's last three waves hold one row, then none
    (129, 129, 1, (1, 2)),  # a second row tile holding one row
    (200, 1000, 48, (1, 3, 16)),  # kv_len % 16 != 0: per-element mask; empty splits
]


@pytest.mark.gpu
@pytest.mark.parametrize("q_len,kv_len,bs,splits", DECODE)
def test_decode_applies_mask_exactly(cuda, q_len, kv_len, bs, splits):
    H = 2
    mask = decode_mask(q_len, kv_len, bs)
    counts = mask.sum(axis=1)
    q = torch.zeros((1, H, q_len, D), device=cuda, dtype=torch.bfloat16)
    k = torch.zeros((1, H, kv_len, D), device=cuda, dtype=torch.bfloat16)
    for name, bucket in BUCKETS.items():
        v = dev(onehot_rows(kv_len, bucket), H, cuda)
        want = histogram(mask, bucket) / counts[:, None]
        for ns in splits:
            print(f"decode mask q_len={q_len} kv_len={kv_len} bs={bs} {name} splits={ns}", flush=True)
            o = splitkv_capi(q, k, v, bs, ns)
            torch.cuda.synchronize()
            got = o[0].double().cpu().numpy()
            err = np.abs(got - want[None])
            assert np.all(got[:, want == 0] == 0), f"{name} splits={ns}: invisible bucket got weight"
            assert np.all(err <= bf16_ulp(want)[None] + 1e-9), \
                f"{name} splits={ns}: max err {err.max()} (worst rel {np.max(err / np.maximum(want, 1e-30))})"
