"""Pins the mask oracle (oracle/mask.py) before anything is checked against
it: brute-force fixtures, the reference's two other statements of the same
mask, closed-form counts, the documented special cases, and the sampling
slice. A planted mistake in a copy of the oracle must fail these pins."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle.mask import block_diff_mask, decode_mask, live_tile_fraction, pair_count

GOLDEN = json.loads((Path(__file__).parent / "golden" / "bd3_golden.json").read_text())


def rows_to_array(rows):
    return np.array([[c == "1" for c in r] for r in rows], dtype=bool)


@pytest.mark.parametrize("case", GOLDEN["train_masks"], ids=lambda c: f"n{c['n']}_bs{c['block_size']}")
def test_train_mask_matches_bruteforce_fixture(case):
    assert np.array_equal(block_diff_mask(case["n"], case["block_size"]), rows_to_array(case["rows"]))


@pytest.mark.parametrize("case", GOLDEN["decode_masks"],
                         ids=lambda c: f"q{c['q_len']}_kv{c['kv_len']}_bs{c['block_size']}")
def test_decode_mask_matches_bruteforce_fixture(case):
    got = decode_mask(case["q_len"], case["kv_len"], case["block_size"])
    assert np.array_equal(got, rows_to_array(case["rows"]))


def flex_mask_mod_statement(n, bs):
    """bench/attention_bench.py:25-38 restated: block ids via where(clean, idx - n, idx)."""
    q = np.arange(2 * n)[:, None]
    k = np.arange(2 * n)[None, :]
    qc, kc = q >= n, k >= n
    qb = np.where(qc, q - n, q) // bs
    kb = np.where(kc, k - n, k) // bs
    return (~qc & ~kc & (qb == kb)) | (~qc & kc & (kb < qb)) | (qc & kc & (kb <= qb))


def triton_statement(n, bs):
    """kernels/BlockSparseFlashAttention.py:12-30 restated (the unused Triton
    bd3lm_mask): mask |= terms in the order written there."""
    q = np.arange(2 * n)[:, None]
    k = np.arange(2 * n)[None, :]
    qc, kc = q >= n, k >= n
    qb, kb = (q % n) // bs, (k % n) // bs
    m = (~qc & ~kc) & (qb == kb)
    m = m | ((~qc & kc) & (qb > kb))
    m = m | ((qc & kc) & (qb >= kb))
    return m


@pytest.mark.parametrize("n,bs", [(8, 1), (8, 3), (16, 4), (64, 16), (96, 7), (128, 128), (256, 64)])
def test_three_statements_agree(n, bs):
    m = block_diff_mask(n, bs)
    assert np.array_equal(m, flex_mask_mod_statement(n, bs))
    assert np.array_equal(m, triton_statement(n, bs))


@pytest.mark.parametrize("n,bs", [(n, bs) for n in (16, 64, 256, 1024) for bs in (1, 2, 4, 16, 64, 256, 1024)
                                  if bs <= n and n % bs == 0])
def test_pair_count_closed_form(n, bs):
    m = block_diff_mask(n, bs)
    assert int(m.sum()) == pair_count(n, bs) == n * n + n * bs
    # density 1/4 + bs/(4n)
    assert abs(m.mean() - (0.25 + bs / (4 * n))) < 1e-12


def test_block_size_n_is_full_attention_per_half():
    """model/bd3lm.py:23: block_size = n reduces the noisy half to full attention."""
    n = 32
    m = block_diff_mask(n, n)
    assert m[:n, :n].all() and not m[:n, n:].any() and m[n:, n:].all() and not m[n:, :n].any()


def test_block_size_1_is_token_causal():
    """model/bd3lm.py:24: block_size = 1 makes the clean half token-causal."""
    n = 32
    m = block_diff_mask(n, 1)
    assert np.array_equal(m[n:, n:], np.tril(np.ones((n, n), dtype=bool)))
    assert np.array_equal(m[:n, :n], np.eye(n, dtype=bool))
    assert np.array_equal(m[:n, n:], np.tril(np.ones((n, n), dtype=bool), k=-1))
    assert not m[n:, :n].any()


@pytest.mark.parametrize("n,bs,L", [(64, 16, 64), (64, 16, 32), (96, 32, 96), (60, 6, 30)])
def test_decode_mask_is_sampling_slice(n, bs, L):
    """The uncached sampler slices attn_mask[n:n+L, n:n+L] (model/bd3lm.py:168);
    the decode kernels' rule over the last q_len rows is that slice."""
    full = block_diff_mask(n, bs)[n:n + L, n:n + L]
    for q_len in (1, bs, L):
        assert np.array_equal(decode_mask(q_len, L, bs), full[L - q_len:])


def test_cached_step_sees_everything():
    """A cached denoising step (q_len = bs, kv_len % bs == 0) is unmasked
    (model/bd3lm.py:184-185)."""
    assert decode_mask(16, 4112, 16).all()
    assert decode_mask(32, 2048, 32).all()


def test_live_tile_fractions_reference_tiling():
    """Live fractions of the reference's 128x64 tiling at its benchmark shapes (configs 1 and 2):
    31.25% of the tiles at n = 1024, bs = 16, and 27-28% at n = 2048."""
    assert abs(live_tile_fraction(block_diff_mask(1024, 16), 128, 64) - 0.3125) < 1e-12
    for bs, frac in ((4, 0.28125), (16, 0.28125), (64, 0.2734375), (256, 0.28125)):
        assert abs(live_tile_fraction(block_diff_mask(2048, bs), 128, 64) - frac) < 1e-12


def test_planted_mistakes_fail_the_pins():
    """Each plausible mistake (offset rule <= instead of <, clean rule <
    instead of <=, dropped diagonal, block id without mod n) breaks at least
    one pin above."""
    n, bs = 8, 2
    q = np.arange(2 * n)[:, None]
    k = np.arange(2 * n)[None, :]
    qc, kc = q >= n, k >= n
    qb, kb = (q % n) // bs, (k % n) // bs
    good = block_diff_mask(n, bs)
    mutants = [
        (~qc & ~kc & (qb == kb)) | (~qc & kc & (kb <= qb)) | (qc & kc & (kb <= qb)),
        (~qc & ~kc & (qb == kb)) | (~qc & kc & (kb < qb)) | (qc & kc & (kb < qb)),
        (~qc & kc & (kb < qb)) | (qc & kc & (kb <= qb)),
        (~qc & ~kc & (q // bs == k // bs)) | (~qc & kc & (k // bs < q // bs)) | (qc & kc & (k // bs <= q // bs)),
    ]
    fixture = next(c for c in GOLDEN["train_masks"] if c["n"] == n and c["block_size"] == bs)
    for mut in mutants:
        assert not np.array_equal(mut, rows_to_array(fixture["rows"]))
        assert int(mut.sum()) != pair_count(n, bs) or not np.array_equal(mut, good)
