"""The C-ABI library on a machine without a GPU: it loads, exports every
symbol include/bd3attn.h declares, its host-only census/classification
agree with the mask oracle, and every precondition violation returns
BD3_EINVAL with a message before any HIP call."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from kernels import _native
from oracle.mask import block_diff_mask

HEADER = Path(__file__).resolve().parent.parent / "include" / "bd3attn.h"


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        import __graft_entry__
        __graft_entry__.build()
    return _native.lib()


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bd3_\w+)\s*\(", text)))


def test_exports_every_declared_symbol(lib):
    names = header_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), f"{name} not exported"
    assert sorted(_native.SIGNATURES) == names, "ctypes table out of sync with the header"


def test_abi_version(lib):
    assert lib.bd3_abi_version() == 2


@pytest.mark.parametrize("n,bs", [(128, 1), (128, 16), (256, 4), (256, 100), (384, 64), (512, 512),
                                  (1024, 16), (2048, 256)])
def test_census_matches_oracle(lib, n, bs):
    out = (ctypes.c_int64 * 8)()
    assert lib.bd3_train_tile_census(n, bs, out) == 0
    m = block_diff_mask(n, bs)
    assert out[0] == int(m.sum())            # useful pairs
    if n % bs == 0:
        assert out[5] == out[0] == n * n + n * bs
    # executed pairs of each schedule recounted from the mask at its granularity:
    # (32 rows x 64 keys) for the forward / dQ, (64 rows x 32 keys) for dK/dV
    rows = m.reshape(2 * n // 32, 32, 2 * n // 64, 64).any(axis=(1, 3))
    keys = m.reshape(2 * n // 64, 64, 2 * n // 32, 32).any(axis=(1, 3))
    blk = m.reshape(2 * n // 32, 32, 2 * n // 32, 32).any(axis=(1, 3))  # live 32 x 32 blocks
    if bs % 16 == 0:  # the backward items skip 32 x 32 blocks with no live pair
        assert out[6] == out[7] == 1024 * int(blk.sum())
    if 32 % bs == 0:  # noisy key tiles: each 32-key wave computes its diagonal 32 x 32 block only
        diag = m[:n, :n].reshape(n // 32, 32, n // 32, 32).any(axis=(1, 3))
        assert np.array_equal(diag, np.eye(n // 32, dtype=bool))
        keys[:, : n // 32] = False
        if bs % 16:
            assert out[7] == 2048 * int(keys.sum()) + 1024 * (n // 32)
        # the forward and the main launch's dQ items: each noisy 32-row wave's one live
        # noisy 64-key tile becomes its diagonal 32 x 32 block
        noisy = rows[: n // 32, : n // 64]
        assert np.array_equal(noisy.sum(axis=1), np.ones(n // 32, dtype=int))
        assert out[1] == 2048 * int(rows.sum()) - 1024 * (n // 32)
        if bs % 16:
            assert out[6] == out[1]
    else:
        assert out[1] == 2048 * int(rows.sum())
        if bs % 16:
            assert out[7] == 2048 * int(keys.sum())
            assert out[6] == out[1]
    assert out[1] >= 1024 * (out[2] + out[3]) >= out[0]


@pytest.mark.parametrize("n,bs", [(64, 1), (64, 16), (96, 7), (128, 32), (128, 128), (160, 64),
                                  (256, 256), (192, 48), (64, 100)])
def test_classification_exact(lib, n, bs):
    """none = no live pair, full = all live, partial = mixed, for every
    (32-row group, 32-key sub-block)."""
    m = block_diff_mask(n, bs)
    for q0 in range(0, 2 * n, 32):
        for k0 in range(0, 2 * n, 32):
            blk = m[q0:q0 + 32, k0:k0 + 32]
            want = 0 if not blk.any() else (1 if blk.all() else 2)
            assert lib.bd3_train_classify(n, bs, q0, k0) == want, (q0, k0)
            assert lib.bd3_train_classify_keys(n, bs, q0, k0) == want, (q0, k0)


def _cls(blk):
    return 0 if not blk.any() else (1 if blk.all() else 2)


@pytest.mark.parametrize("n,bs", [(128, 1), (128, 16), (128, 100), (256, 7), (256, 48), (384, 64),
                                  (512, 512), (1024, 16), (640, 33)])
@pytest.mark.parametrize("mode", [0, 1])
def test_walk_classes_match_mask(lib, n, bs, mode):
    """Per-tile classes in walk-index interval form (the forward kernel's
    whole-tile classes are mode 0) against the mask. mode 0: 32-row groups
    walking the key tiles of their 128-row query tile; mode 1: 32-key groups
    walking the query tiles of their 128-key tile. The walk visits
    distinct tiles and every tile where the 128-wide tile has a live pair;
    each tile of it is none / full / partial for the group exactly as the
    group's 32 x 64 mask block is, and so is each 32 x 32 half."""
    m = block_diff_mask(n, bs)
    if mode == 1:
        m = m.T  # rows <-> keys: a key group's view of the queries
    tile = ctypes.c_int32()
    for g0 in range(0, 2 * n, 32):
        walk, classes = [], []
        while True:
            c = lib.bd3_train_walk_class(n, bs, g0, len(walk), mode, ctypes.byref(tile))
            if c == -3:
                break
            assert c >= 0, (g0, c)
            walk.append(tile.value)
            classes.append(c)
        assert len(set(walk)) == len(walk), (g0, walk)
        r0 = g0 - g0 % 128
        need = {t for t in range(2 * n // 64) if m[r0:r0 + 128, 64 * t:64 * t + 64].any()}
        assert need <= set(walk), (g0, sorted(need - set(walk)))
        for t, c in zip(walk, classes):
            blk = m[g0:g0 + 32, 64 * t:64 * t + 64]
            want = _cls(blk) | _cls(blk[:, :32]) << 2 | _cls(blk[:, 32:]) << 4
            assert c == want, (g0, t, c, want)
    assert lib.bd3_train_walk_class(n, bs, 0, 10 ** 6, mode, ctypes.byref(tile)) == -3
    assert lib.bd3_train_walk_class(n, bs, 16, 0, mode, ctypes.byref(tile)) == -1
    assert lib.bd3_train_walk_class(n, bs, 0, 0, mode, None) == -1
    assert lib.bd3_train_walk_class(n, bs, 0, 0, 2, ctypes.byref(tile)) == -1


@pytest.mark.parametrize("n,bs", [(8, 1), (8, 3), (64, 16), (96, 7), (128, 128), (256, 64)])
def test_interval_forms_match_mask(lib, n, bs):
    """The row intervals (forward, dQ items) and column intervals (dK/dV
    items) reproduce every row and column of block_diff_mask."""
    m = block_diff_mask(n, bs)
    out = (ctypes.c_int32 * 4)()
    idx = np.arange(2 * n)
    for i in range(2 * n):
        for mode, want in ((0, m[i, :]), (1, m[:, i])):
            assert lib.bd3_train_intervals(n, bs, i, mode, out) == 0
            lo1, hi1, lo2, hi2 = list(out)
            got = ((idx >= lo1) & (idx < hi1)) | ((idx >= lo2) & (idx < hi2))
            assert np.array_equal(got, want), (mode, i)


def _i64(vals):
    return (ctypes.c_int64 * len(vals))(*vals)


GOOD = 0x100000  # a 16-byte aligned fake device address: never dereferenced,
                 # every call below fails validation before any HIP call


def expect_einval(status, fragment):
    assert status == _native.BD3_EINVAL
    assert fragment in _native.last_error()


def test_fwd_validation(lib):
    st = _i64([8 * 64 * 256] * 0 + [64 * 256, 64 * 256, 64] * 4)
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, GOOD, 1, 1, 100, 64, 16, st, 0.125, None),
                  "multiple of 128")
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, GOOD, 1, 1, 128, 128, 16, st, 0.125, None),
                  "head_dim")
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, GOOD, 1, 1, 128, 64, 0, st, 0.125, None),
                  "block_size")
    expect_einval(lib.bd3_attn_fwd(None, GOOD, GOOD, GOOD, GOOD, 1, 1, 128, 64, 16, st, 0.125, None),
                  "q is NULL")
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD + 2, GOOD, GOOD, GOOD, 1, 1, 128, 64, 16, st, 0.125, None),
                  "aligned")
    bad = _i64([64 * 256, 64 * 256, 63] + [64 * 256, 64 * 256, 64] * 3)
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, GOOD, 1, 1, 128, 64, 16, bad, 0.125, None),
                  "stride")
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, None, 1, 1, 128, 64, 16, st, 0.125, None),
                  "lse")


def test_bwd_validation(lib):
    st = _i64([64 * 256, 64 * 256, 64] * 8)
    need = lib.bd3_attn_bwd_workspace_bytes(1, 1, 128, 64)
    assert need == 2 * 1 * 1 * 256 * 4  # Delta and -L / scale
    args = [GOOD] * 9
    expect_einval(lib.bd3_attn_bwd(*args, GOOD, need, 1, 1, 128, 64, 3, st, 0.125, None), "multiple of block_size")
    expect_einval(lib.bd3_attn_bwd(*args, GOOD, need - 1, 1, 1, 128, 64, 16, st, 0.125, None), "workspace")
    expect_einval(lib.bd3_attn_bwd(*args, None, need, 1, 1, 128, 64, 16, st, 0.125, None), "workspace")
    st18 = _i64([64 * 256, 64 * 256, 64] * 6)
    expect_einval(lib.bd3_attn_bwd_dq(*[GOOD] * 7, None, 1, 1, 128, 64, 16, st18, 0.125, None), "delta")
    expect_einval(lib.bd3_attn_bwd_dkdv(*[GOOD] * 8, 1, 1, 128, 64, 5, st18, 0.125, None), "block_size")
    expect_einval(lib.bd3_attn_bwd_dkdv(GOOD, GOOD, GOOD, GOOD + 8, *[GOOD] * 4, 1, 1, 128, 64, 16, st18,
                                        0.125, None), "dout")


def test_bwd_stage_validation(lib):
    """The Delta pass and the main launch refuse bad arguments before any
    HIP call (fake device pointers)."""
    st6, st21 = _i64([64 * 256, 64 * 256, 64] * 2), _i64([64 * 256, 64 * 256, 64] * 7)
    expect_einval(lib.bd3_attn_bwd_delta(GOOD, GOOD, GOOD, None, 1, 1, 128, 64, 16, st6, 0.125, None), "delta")
    expect_einval(lib.bd3_attn_bwd_delta(GOOD, GOOD + 8, GOOD, GOOD, 1, 1, 128, 64, 16, st6, 0.125, None), "dout")
    expect_einval(lib.bd3_attn_bwd_delta(GOOD, GOOD, GOOD, GOOD, 1, 1, 100, 64, 16, st6, 0.125, None), "multiple of 128")
    expect_einval(lib.bd3_attn_bwd_main(*[GOOD] * 5, None, *[GOOD] * 3, 1, 1, 128, 64, 16, st21, 0.125, None), "delta")
    expect_einval(lib.bd3_attn_bwd_main(*[GOOD] * 9, 1, 1, 128, 64, 5, st21, 0.125, None), "block_size")
    bad = [64 * 256, 64 * 256, 64] * 7
    bad[3 * 3 + 2] = 1 << 24  # dout's sequence stride: loaded tile by tile
    expect_einval(lib.bd3_attn_bwd_main(*[GOOD] * 9, 1, 1, 128, 64, 16, _i64(bad), 0.125, None), "dout sequence stride")
    for scale in (0.0, float("nan")):
        expect_einval(lib.bd3_attn_bwd_delta(*[GOOD] * 4, 1, 1, 128, 64, 16, st6, scale, None), "scale")
        expect_einval(lib.bd3_attn_bwd_main(*[GOOD] * 9, 1, 1, 128, 64, 16, st21, scale, None), "scale")


def test_bwd_refuses_before_any_launch(lib):
    """bd3_attn_bwd checks the direct-load stride limit of both stages' tile
    operands (dQ: k, v; dK/dV: q, dout) before its first launch, so a refused
    call has written nothing (fake device pointers, no GPU needed)."""
    need = lib.bd3_attn_bwd_workspace_bytes(1, 1, 128, 64)
    for slot, name in ((0, "q"), (1, "k"), (2, "v"), (4, "dout")):
        st = [64 * 256, 64 * 256, 64] * 8
        st[3 * slot + 2] = 1 << 24
        expect_einval(lib.bd3_attn_bwd(*[GOOD] * 9, GOOD, need, 1, 1, 128, 64, 16, _i64(st), 0.125, None),
                      f"{name} sequence stride")


@pytest.mark.parametrize("scale", [0.0, -0.125, float("nan"), float("inf")])
def test_scale_validation(lib, scale):
    """The kernels take row maxima over the raw scores and scale them
    afterwards: every attention entry point rejects a scale that is not
    finite and positive."""
    st = _i64([64 * 256, 64 * 256, 64] * 4)
    expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, GOOD, 1, 1, 128, 64, 16, st, scale, None), "scale")
    st24 = _i64([64 * 256, 64 * 256, 64] * 8)
    need = lib.bd3_attn_bwd_workspace_bytes(1, 1, 128, 64)
    expect_einval(lib.bd3_attn_bwd(*[GOOD] * 9, GOOD, need, 1, 1, 128, 64, 16, st24, scale, None), "scale")
    expect_einval(lib.bd3_attn_bwd_noalloc(*[GOOD] * 9, 1, 1, 128, 64, 16, st24, scale, None), "scale")
    st18 = _i64([64 * 256, 64 * 256, 64] * 6)
    expect_einval(lib.bd3_attn_bwd_dq(*[GOOD] * 8, 1, 1, 128, 64, 16, st18, scale, None), "scale")
    expect_einval(lib.bd3_attn_bwd_dkdv(*[GOOD] * 8, 1, 1, 128, 64, 16, st18, scale, None), "scale")
    sd = _i64([64 * 256, 64 * 256, 64] * 4)
    expect_einval(lib.bd3_decode(GOOD, GOOD, GOOD, GOOD, 1, 1, 16, 256, 64, 16, sd, scale, GOOD, 1 << 20, None),
                  "scale")
    expect_einval(lib.bd3_decode_splitkv(GOOD, GOOD, GOOD, GOOD, 1, 1, 16, 256, 64, 16, 2, sd, scale, GOOD,
                                         1 << 20, None), "scale")


def test_tile_load_offset_stride_limit(lib):
    """Sequence strides of the tensors the training kernels load tile by tile
    (k, v in the forward and the dQ items; q, dO in dK/dV) must keep the 32-bit
    per-lane load offsets in range: < 2^24 elements."""
    big = 1 << 24
    ok = [64 * 256, 64 * 256, 64]
    for slot, name in ((1, "k"), (2, "v")):
        st = [*ok * 4]
        st[3 * slot + 2] = big
        expect_einval(lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, GOOD, 1, 1, 128, 64, 16, _i64(st), 0.125, None),
                      f"{name} sequence stride")
        st18 = [*ok * 6]
        st18[3 * slot + 2] = big
        expect_einval(lib.bd3_attn_bwd_dq(*[GOOD] * 8, 1, 1, 128, 64, 16, _i64(st18), 0.125, None),
                      f"{name} sequence stride")
    for slot, name in ((0, "q"), (3, "dout")):
        st18 = [*ok * 6]
        st18[3 * slot + 2] = big
        expect_einval(lib.bd3_attn_bwd_dkdv(*[GOOD] * 8, 1, 1, 128, 64, 16, _i64(st18), 0.125, None),
                      f"{name} sequence stride")
    # decode with q_len > 64 runs the prefill kernel, which loads k and v tile by tile
    for slot, name in ((1, "k"), (2, "v")):
        st = [64 * 4096, 64 * 4096, 64] * 4
        st[3 * slot + 2] = big
        expect_einval(lib.bd3_decode_splitkv(GOOD, GOOD, GOOD, GOOD, 1, 1, 65, 4096, 64, 16, 1, _i64(st), 0.125,
                                             None, 0, None), f"{name} sequence stride")
    # q's stride in the forward is not a tile-load offset: only the 8-alignment applies
    st = [big - 8, 64, 64] + ok * 3
    status = lib.bd3_attn_fwd(GOOD, GOOD, GOOD, GOOD, None, 1, 1, 128, 64, 16, _i64(st), 0.125, None)
    expect_einval(status, "lse")  # passed the stride checks, stopped at the next one


def test_decode_validation(lib):
    st = _i64([64 * 64, 64 * 64, 64] * 4)
    expect_einval(lib.bd3_decode(GOOD, GOOD, GOOD, GOOD, 1, 1, 33, 32, 64, 16, st, 0.125, GOOD, 0, None),
                  "q_len")
    expect_einval(lib.bd3_decode_splitkv(GOOD, GOOD, GOOD, GOOD, 1, 1, 16, 32, 64, 16, 0, st, 0.125, GOOD,
                                         1 << 20, None), "n_splits")
    expect_einval(lib.bd3_decode_splitkv(GOOD, GOOD, GOOD, GOOD, 1, 1, 16, 32, 64, 16, 33, st, 0.125, GOOD,
                                         1 << 20, None), "n_splits")
    need = lib.bd3_decode_workspace_bytes(1, 1, 16, 32, 64, 2)
    expect_einval(lib.bd3_decode_splitkv(GOOD, GOOD, GOOD, GOOD, 1, 1, 16, 32, 64, 16, 2, st, 0.125, GOOD,
                                         need - 1, None), "workspace")
    expect_einval(lib.bd3_mask_dump(GOOD, 2, 4, 4, 1, None), "mode")
    expect_einval(lib.bd3_mask_dump(GOOD, 1, 5, 4, 1, None), "q_len")


def test_clock_probe_validation(lib):
    rate = ctypes.c_int64(0)
    expect_einval(lib.bd3_clock_probe(None, 4, 10, ctypes.byref(rate), None), "NULL")
    expect_einval(lib.bd3_clock_probe(GOOD, 0, 10, ctypes.byref(rate), None), "workgroups")
    expect_einval(lib.bd3_clock_probe(GOOD, 65537, 10, ctypes.byref(rate), None), "workgroups")
    expect_einval(lib.bd3_clock_probe(GOOD, 4, 0, ctypes.byref(rate), None), "iters")
    expect_einval(lib.bd3_clock_probe(GOOD, 4, 10, None, None), "NULL")


def test_workspace_sizes(lib):
    # one split needs no workspace; partials are (BH, q_tiles, splits, 32, 64) fp32 + LSE
    assert lib.bd3_decode_workspace_bytes(2, 3, 16, 100, 64, 1) == 0
    slots = 2 * 3 * 1 * 4 * 32
    assert lib.bd3_decode_workspace_bytes(2, 3, 16, 100, 64, 4) == slots * 64 * 4 + ((slots * 4 + 255) // 256) * 256
    s = lib.bd3_decode_auto_splits(32, 12, 16, 4112)
    assert s == 1  # 384 workgroups at one split already cover 256 CUs
    # 96 (b, h) x 1 32-row tile: about 128 workgroups, at least 1024 keys per
    # split with 64 or more tiles (512 with fewer)
    assert [lib.bd3_decode_auto_splits(8, 12, 32, kv) for kv in (100, 544, 1056, 2080, 4096)] == [1, 1, 1, 2, 2]
    assert lib.bd3_decode_auto_splits(1, 12, 32, 3584) == 7
    # a cached step (q_len <= 16): down to 128 keys per split, at most 16 splits
    assert [lib.bd3_decode_auto_splits(1, 12, 16, kv) for kv in (200, 544, 3584, 8192)] == [1, 4, 16, 16]
    assert lib.bd3_decode_auto_splits(2, 12, 16, 1024) == 8
    # q_len > 64 (the prefill kernel): no split once the items fill half the
    # 1024 workgroup slots, else split only until the longest item is no
    # longer than the whole grid's share per slot allows
    assert lib.bd3_decode_auto_splits(1, 12, 3088, 3088) == 4
    assert lib.bd3_decode_auto_splits(8, 12, 2048, 2048) == 1
    assert lib.bd3_decode_auto_splits(8, 12, 1024, 1024) == 1  # 768 items
    assert lib.bd3_decode_auto_splits(1, 12, 8192, 8192) == 1  # 768 items
    assert lib.bd3_decode_auto_splits(32, 12, 128, 4112) == 2  # 384 items
    assert lib.bd3_decode_auto_splits(4, 12, 256, 4096) == 6
    assert lib.bd3_decode_auto_splits(1, 12, 128, 3584) == 14
    assert lib.bd3_decode_workspace_bytes(32, 12, 16, 4112, 64, 0) == lib.bd3_decode_workspace_bytes(
        32, 12, 16, 4112, 64, s)


def test_qkv_rope_validation(lib):
    xs = _i64([32 * 2304, 2304])
    os_ = _i64([12 * 32 * 64, 32 * 64, 64] * 3)
    call = lambda **kw: lib.bd3_qkv_rope(
        kw.get("qkv", GOOD), kw.get("xs", xs), kw.get("batch", 2), kw.get("seq", 32), 12,
        kw.get("d", 64), kw.get("positions", None), kw.get("pos0", 0), kw.get("sin", GOOD), GOOD,
        kw.get("max_pos", 2048), kw.get("q", GOOD), GOOD, GOOD, kw.get("os", os_), None)
    expect_einval(call(d=128), "head_dim must be 64")
    expect_einval(call(batch=0), "batch >= 1")
    expect_einval(call(seq=-1), "seq >= 0")
    expect_einval(call(qkv=GOOD + 2), "16-byte aligned")
    expect_einval(call(xs=_i64([32 * 2304, 2300])), "qkv stride[1]")
    expect_einval(call(sin=None), "sin_table")
    expect_einval(call(max_pos=0), "max_pos")
    expect_einval(call(pos0=2040), "exceed the RoPE table")
    expect_einval(call(pos0=-1), "exceed the RoPE table")
    expect_einval(call(q=None), "q_out is NULL")
    expect_einval(call(os=_i64([12 * 32 * 64, 32 * 64, 60] + [0, 0, 64] * 2)), "q_out stride[2]")


def test_kv_write_validation(lib):
    st = _i64([12 * 32 * 64, 32 * 64, 64] * 4)
    expect_einval(lib.bd3_kv_write(GOOD, GOOD, GOOD, GOOD, 1, 12, 32, 32, st, None), "head_dim must be 64")
    expect_einval(lib.bd3_kv_write(GOOD, GOOD, None, GOOD, 1, 12, 32, 64, st, None), "k_dst is NULL")
    expect_einval(lib.bd3_kv_write(GOOD, GOOD, GOOD, GOOD, 1, 12, -2, 64, st, None), "seq >= 0")
    expect_einval(lib.bd3_kv_write(GOOD, GOOD, GOOD, GOOD, 1, 12, 32, 64, None, None), "strides is NULL")


def test_subs_sample_validation(lib):
    ok = dict(logits=GOOD, ld=1000, fp32=0, xt=GOOD, out=GOOD, rows=4, vocab=1000, mask=999, keep=0.5)

    def call(**kw):
        a = {**ok, **kw}
        return lib.bd3_subs_sample(a["logits"], a["ld"], a["fp32"], a["xt"], a["out"], a["rows"], a["vocab"],
                                   a["mask"], a["keep"], None, 0, 0, None)
    expect_einval(call(vocab=1), "vocab must be >= 2")
    expect_einval(call(mask=1000), "mask_index 1000 outside")
    expect_einval(call(mask=-1), "mask_index -1 outside")
    expect_einval(call(ld=999), "row stride ld")
    expect_einval(call(fp32=2), "logits_fp32")
    expect_einval(call(keep=1.5), "keep (s / t)")
    expect_einval(call(keep=float("nan")), "keep (s / t)")
    expect_einval(call(xt=None), "non-NULL")
    expect_einval(call(rows=-1), "rows must be >= 0")


def test_dit_glue_validation(lib):
    st5 = _i64([768 * 16, 768, 768, 768 * 16, 768])
    st7 = _i64([768 * 16, 768, 768, 768 * 16, 768, 768 * 16, 768])
    ln = lambda **kw: lib.bd3_ln_modulate(kw.get("x", GOOD), kw.get("xf", 1), GOOD, 1, GOOD, GOOD, kw.get("mf", 0),
                                          GOOD, kw.get("of", 1), 2, 16, kw.get("d", 768), kw.get("st", st5),
                                          kw.get("eps", 1e-5), None)
    expect_einval(ln(d=100), "multiple of 8")
    expect_einval(ln(x=GOOD + 8), "x must be 16-byte aligned")
    expect_einval(ln(xf=2), "dtype flags")
    expect_einval(ln(xf=0, mf=0, of=1), "out must be bf16")
    expect_einval(ln(st=_i64([768 * 16, 770, 768, 768 * 16, 768])), "stride[1]")
    expect_einval(ln(eps=-1.0), "eps")
    gr = lambda **kw: lib.bd3_gate_residual(GOOD, 1, kw.get("g", GOOD), 0, GOOD, 0, GOOD, 2, 16, kw.get("d", 768),
                                            kw.get("st", st7), None)
    expect_einval(gr(g=None), "gate is NULL")
    expect_einval(gr(d=0), "multiple of 8")
    expect_einval(gr(st=None), "strides is NULL")


def test_fused_glue_validation(lib):
    st9 = _i64([768 * 16, 768, 768 * 6, 768 * 16, 768, 768 * 16, 768, 768 * 16, 768])
    fu = lambda **kw: lib.bd3_gate_residual_ln_modulate(
        GOOD, kw.get("xf", 0), kw.get("g", GOOD), GOOD, kw.get("yf", 0), kw.get("xo", GOOD), GOOD, 1, GOOD, GOOD,
        kw.get("mf", 0), GOOD, kw.get("of", 0), 2, 16, kw.get("d", 768), kw.get("st", st9), kw.get("eps", 1e-5), None)
    expect_einval(fu(g=None), "gate is NULL")
    expect_einval(fu(xo=GOOD + 8), "x_out must be 16-byte aligned")
    expect_einval(fu(d=4104), "d_model must be <= 4096")
    expect_einval(fu(of=1), "out must be bf16")   # all bf16: modulates in bf16
    expect_einval(fu(yf=3), "dtype flags")
    expect_einval(fu(eps=float("nan")), "eps")
    expect_einval(fu(st=_i64([768 * 16, 768, 768 * 6, 768 * 16, 768, 768 * 16, 769, 768 * 16, 768])), "stride[6]")
