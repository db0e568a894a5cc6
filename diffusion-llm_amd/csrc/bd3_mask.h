// bd3_mask.h - integer-only BD3-LM mask predicates and tile classification,
// shared by the gfx950 kernels and the host (C-ABI census helpers, CPU tests).
//
// Training layout: the attention sequence is cat(x_t, x_0) of length 2n.
// Index < n is the noisy copy x_t, index >= n the clean copy x_0; the block id
// of an index is (index mod n) / bs. Rules (model/bd3lm.py:17-21, :41-52):
//   noisy row, block b -> noisy keys of block b          (block diagonal)
//   noisy row, block b -> clean keys of blocks < b       (offset block-causal)
//   clean row, block b -> clean keys of blocks <= b      (block-causal)
//   clean row          -> noisy keys: never
// The same predicate is stated by the FlexAttention mask_mod
// (bench/attention_bench.py:25-38) and the Triton bd3lm_mask
// (kernels/BlockSparseFlashAttention.py:12-30).
//
// Decode layout: queries are the last q_len of kv_len positions; row i sits
// at position p = kv_len - q_len + i and sees key j iff j / bs <= p / bs and
// j < kv_len (kernels/BlockSparseDecodeAttention.py:84-88, :23-26), i.e. the
// clean-clean quadrant of the training mask sliced as model/bd3lm.py:168.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define BD3_HD __host__ __device__ __forceinline__
#else
#define BD3_HD static inline
#endif

namespace bd3 {

BD3_HD int imin(int a, int b) { return a < b ? a : b; }
BD3_HD int imax(int a, int b) { return a > b ? a : b; }

// Training mask: may row q attend to key k (both in [0, 2n))?
BD3_HD bool train_visible(int q, int k, int n, int bs) {
  const bool qc = q >= n, kc = k >= n;
  const int qb = (qc ? q - n : q) / bs;
  const int kb = (kc ? k - n : k) / bs;
  if (!qc && !kc) return qb == kb;
  if (!qc && kc) return kb < qb;
  if (qc && kc) return kb <= qb;
  return false;
}

// Decode mask: may query row i (of q_len, the last positions) attend to key j?
BD3_HD bool decode_visible(int i, int j, int q_len, int kv_len, int bs) {
  const int p = kv_len - q_len + i;
  return j < kv_len && (j / bs) <= (p / bs);
}

// Visible-key count of one training row (its live pairs), for the census.
// Noisy row of block b: its own block [bs*b, min(bs*(b+1), n)) plus the bs*b
// earlier clean keys; clean row of block b: min(bs*(b+1), n) clean keys.
BD3_HD int train_row_keys(int q, int n, int bs) {
  const int b = (q < n ? q : q - n) / bs;
  return imin(bs * (b + 1), n);
}

// The keys one training row sees, as two half-open intervals of global key
// indices: key k is visible iff lo1 <= k < hi1 or lo2 <= k < hi2. Equivalent
// to train_visible(q, k, n, bs) for every k in [0, 2n).
struct RowIntervals {
  int lo1, hi1, lo2, hi2;
};

BD3_HD RowIntervals train_row_intervals(int q, int n, int bs) {
  RowIntervals r;
  if (q < n) {
    const int b = q / bs;
    r.lo1 = bs * b;
    r.hi1 = imin(bs * (b + 1), n);
    r.lo2 = n;
    r.hi2 = n + bs * b;
  } else {
    const int b = (q - n) / bs;
    r.lo1 = n;
    r.hi1 = n + imin(bs * (b + 1), n);
    r.lo2 = 0;
    r.hi2 = 0;
  }
  return r;
}

// Rows that see training key k (global index), as two half-open row
// intervals: the transpose of train_row_intervals.
//   noisy key, block b: noisy rows of block b;
//   clean key, block b: noisy rows of blocks > b and clean rows of blocks >= b.
BD3_HD RowIntervals train_col_intervals(int k, int n, int bs) {
  RowIntervals r;
  if (k < n) {
    const int b = k / bs;
    r.lo1 = bs * b;
    r.hi1 = imin(bs * (b + 1), n);
    r.lo2 = 0;
    r.hi2 = 0;
  } else {
    const int b = (k - n) / bs;
    r.lo1 = imin(bs * (b + 1), n);
    r.hi1 = n;
    r.lo2 = n + bs * b;
    r.hi2 = 2 * n;
  }
  return r;
}

BD3_HD bool row_sees(const RowIntervals& r, int k) {
  return (k >= r.lo1 && k < r.hi1) || (k >= r.lo2 && k < r.hi2);
}

enum TileClass { kNone = 0, kFull = 1, kPartial = 2 };

// Classification of the pairs (rows [q0, q0+R), keys [k0, k0+C)) under the
// training mask. Rows must lie in one half and keys in one half (true for
// 32-aligned groups when n % 32 == 0). kNone and kFull are exact; kPartial
// means some but not all pairs are live.
//
// A kernel that classifies many key groups against one fixed row group
// precomputes the row group's bounds once (RowGroup: no division per tile);
// a kernel with a fixed key group classifies row groups with KeyGroup.
struct RowGroup {
  int clean;      // rows in the clean half
  int diag_lo;    // noisy rows: keys [diag_lo, diag_hi) hold their own blocks
  int diag_hi;
  int one_block;  // noisy rows all in one block
  int full_end;   // clean-key offsets [0, full_end) are seen by every row
  int live_end;   // clean-key offsets >= live_end are seen by no row
};

BD3_HD RowGroup train_row_group(int q0, int R, int n, int bs) {
  RowGroup g;
  g.clean = q0 >= n;
  const int r0 = g.clean ? q0 - n : q0;
  const int b0 = r0 / bs, b1 = (r0 + R - 1) / bs;
  g.diag_lo = bs * b0;
  g.diag_hi = imin(bs * (b1 + 1), n);
  g.one_block = b0 == b1;
  if (g.clean) {  // row in block b sees clean keys [0, min(bs*(b+1), n))
    g.full_end = imin(bs * (b0 + 1), n);
    g.live_end = imin(bs * (b1 + 1), n);
  } else {        // row in block b sees clean keys [0, bs*b)
    g.full_end = bs * b0;
    g.live_end = bs * b1;
  }
  return g;
}

// Written with non-short-circuit operators so that, with a wave-uniform
// RowGroup, the device code is a few scalar compares and selects, no branches.
BD3_HD int row_group_class(const RowGroup& g, int k0, int C, int n) {
  const bool kc = k0 >= n;
  const int a = kc ? k0 - n : k0;  // key offset inside its half
  const int e = a + C;
  // noisy keys: clean rows never see them; noisy rows see their own blocks
  const bool nz_dead = (g.clean != 0) | (e <= g.diag_lo) | (a >= g.diag_hi);
  const bool nz_full = (g.one_block != 0) & (g.diag_lo <= a) & (e <= g.diag_hi);
  // clean keys: a prefix seen by every row, then a partial band
  const bool cl_dead = a >= g.live_end;
  const bool cl_full = e <= g.full_end;
  const bool dead = kc ? cl_dead : nz_dead;
  const bool full = kc ? cl_full : nz_full;
  return dead ? kNone : (full ? kFull : kPartial);
}

BD3_HD int train_class(int q0, int R, int k0, int C, int n, int bs) {
  return row_group_class(train_row_group(q0, R, n, bs), k0, C, n);
}

// The transpose: a fixed key group [k0, k0+C) classified against row groups.
struct KeyGroup {
  int clean;        // keys in the clean half
  int noisy_lo;     // noisy keys: noisy rows [noisy_lo, noisy_hi) hold their blocks
  int noisy_hi;
  int one_block;    // keys all in one block
  int nz_live_lo;   // clean keys: noisy rows >= nz_live_lo see some key,
  int nz_full_lo;   //   noisy rows >= nz_full_lo see every key (row offsets)
  int cl_live_lo;   //   clean row offsets >= cl_live_lo see some key,
  int cl_full_lo;   //   clean row offsets >= cl_full_lo see every key
};

BD3_HD KeyGroup train_key_group(int k0, int C, int n, int bs) {
  KeyGroup g;
  g.clean = k0 >= n;
  const int a0 = g.clean ? k0 - n : k0;
  const int kb0 = a0 / bs, kb1 = (a0 + C - 1) / bs;
  g.noisy_lo = bs * kb0;
  g.noisy_hi = imin(bs * (kb1 + 1), n);
  g.one_block = kb0 == kb1;
  // noisy row of block b sees clean key block kb iff b > kb
  g.nz_live_lo = imin(bs * (kb0 + 1), n);
  g.nz_full_lo = imin(bs * (kb1 + 1), n);
  // clean row of block b sees clean key block kb iff b >= kb
  g.cl_live_lo = bs * kb0;
  g.cl_full_lo = bs * kb1;
  return g;
}

// Branch-free like row_group_class.
BD3_HD int key_group_class(const KeyGroup& g, int q0, int R, int n) {
  const bool qc = q0 >= n;
  const int r = qc ? q0 - n : q0;  // row offset inside its half
  const int e = r + R;
  // noisy keys: clean rows never see them; noisy rows of the same blocks do
  const bool nz_dead = qc | (e <= g.noisy_lo) | (r >= g.noisy_hi);
  const bool nz_full = (g.one_block != 0) & (g.noisy_lo <= r) & (e <= g.noisy_hi);
  // clean keys: rows from live_lo on see some key, from full_lo on all keys
  const int live_lo = qc ? g.cl_live_lo : g.nz_live_lo;
  const int full_lo = qc ? g.cl_full_lo : g.nz_full_lo;
  const int row_end = qc ? e : imin(e, n);
  const bool cl_dead = (row_end <= live_lo) | (!qc & (r >= n));
  const bool cl_full = r >= full_lo;
  const bool dead = g.clean ? cl_dead : nz_dead;
  const bool full = g.clean ? cl_full : nz_full;
  return dead ? kNone : (full ? kFull : kPartial);
}

// The classes of one fixed group (rows for RowGroup, keys for KeyGroup)
// against blocks [p, p+C) of the other axis, as thresholds in absolute
// positions per half (index 0: p < n, 1: p >= n). A block inside one half is
// dead unless p + C > lo and p < hi, and otherwise full iff p >= flo and
// p + C <= fhi. Same answers as row_group_class / key_group_class for that
// group (checked against the mask on the host), at a few scalar compares per
// block once the bounds are in registers.
struct ClassBounds {
  int lo[2], hi[2], flo[2], fhi[2];
};

constexpr int kBoundBig = 1 << 30;

BD3_HD ClassBounds row_group_bounds(const RowGroup& g, int n) {
  ClassBounds b;
  // noisy keys: clean rows see none; noisy rows see their own blocks
  b.lo[0] = g.clean ? kBoundBig : g.diag_lo;
  b.hi[0] = g.diag_hi;
  b.flo[0] = g.one_block ? g.diag_lo : kBoundBig;
  b.fhi[0] = g.diag_hi;
  // clean keys: offsets [0, full_end) seen by all rows, none from live_end
  b.lo[1] = 0;
  b.hi[1] = n + g.live_end;
  b.flo[1] = 0;
  b.fhi[1] = n + g.full_end;
  return b;
}

BD3_HD ClassBounds key_group_bounds(const KeyGroup& g, int n) {
  ClassBounds b;
  if (!g.clean) {  // noisy keys: seen by the noisy rows of their own blocks only
    b.lo[0] = g.noisy_lo;
    b.hi[0] = g.noisy_hi;
    b.flo[0] = g.one_block ? g.noisy_lo : kBoundBig;
    b.fhi[0] = g.noisy_hi;
    b.lo[1] = kBoundBig;
    b.hi[1] = 2 * n;
    b.flo[1] = kBoundBig;
    b.fhi[1] = 2 * n;
  } else {  // clean keys: noisy rows of later blocks, clean rows of this and later blocks
    b.lo[0] = g.nz_live_lo >= n ? kBoundBig : g.nz_live_lo;
    b.hi[0] = n;
    b.flo[0] = g.nz_full_lo;
    b.fhi[0] = n;
    b.lo[1] = n + g.cl_live_lo;
    b.hi[1] = 2 * n;
    b.flo[1] = n + g.cl_full_lo;
    b.fhi[1] = 2 * n;
  }
  return b;
}

BD3_HD int bounds_class(const ClassBounds& b, int p, int C, int n) {
  const int h = p >= n;
  const bool live = (p + C > b.lo[h]) & (p < b.hi[h]);
  const bool full = (p >= b.flo[h]) & (p + C <= b.fhi[h]);
  return live ? (full ? kFull : kPartial) : kNone;
}

// Floor and ceiling of a / b for b > 0 and any sign of a.
BD3_HD int floor_div(int a, int b) { return a >= 0 ? a / b : -((b - 1 - a) / b); }
BD3_HD int ceil_div(int a, int b) { return -floor_div(-a, b); }

// The classes of the tiles of a walk for one fixed group, as intervals of the
// walk index. The walk visits tiles t0 .. t0 + n_first - 1 (walk index
// i = 0 .. n_first - 1), then t2 .. t2 + n_second - 1 (i = n_first ..); each
// range lies in one half. The classified positions of tile t are
// [t * tile + off, t * tile + off + C) (the whole tile, or one 32-wide half
// of it). Tile i is live iff i - live_lo[r] < live_len[r] and full iff
// i - full_lo[r] < full_len[r] (unsigned differences), r = 0 in the first
// range and 1 in the second: the same classes as bounds_class(b, t * tile +
// off, C, n), at a few scalar operations per tile.
struct WalkClasses {
  int live_lo[2], live_len[2], full_lo[2], full_len[2];
};

BD3_HD WalkClasses walk_classes(const ClassBounds& b, int t0, int n_first, int t2, int n_second, int n,
                                int tile, int off, int C) {
  WalkClasses w;
  const int ta[2] = {t0, t2}, cnt[2] = {n_first, n_second};
  int base = 0;
  for (int r = 0; r < 2; ++r) {
    const int h = ta[r] * tile + off >= n;
    // p = t * tile + off: live iff p + C > lo and p < hi; full iff p >= flo
    // and p + C <= fhi.
    const int l0 = floor_div(b.lo[h] - off - C, tile) + 1, l1 = ceil_div(b.hi[h] - off, tile);
    const int f0 = ceil_div(b.flo[h] - off, tile), f1 = floor_div(b.fhi[h] - off - C, tile) + 1;
    // walk indices, clipped to the range; full tiles are live tiles
    const int li0 = imin(imax(l0 - ta[r], 0), cnt[r]), li1 = imin(imax(l1 - ta[r], 0), cnt[r]);
    const int fi0 = imax(imin(imax(f0 - ta[r], 0), cnt[r]), li0);
    const int fi1 = imin(imin(imax(f1 - ta[r], 0), cnt[r]), li1);
    w.live_lo[r] = base + li0;
    w.live_len[r] = imax(li1 - li0, 0);
    w.full_lo[r] = base + fi0;
    w.full_len[r] = imax(fi1 - fi0, 0);
    base += cnt[r];
  }
  return w;
}

// Whether walk tile i is live / full under w (scalar code for a uniform w).
BD3_HD bool walk_live(const WalkClasses& w, int i, int n_first) {
  const bool r0 = i < n_first;
  return (unsigned)(i - (r0 ? w.live_lo[0] : w.live_lo[1])) < (unsigned)(r0 ? w.live_len[0] : w.live_len[1]);
}
BD3_HD bool walk_full(const WalkClasses& w, int i, int n_first) {
  const bool r0 = i < n_first;
  return (unsigned)(i - (r0 ? w.full_lo[0] : w.full_lo[1])) < (unsigned)(r0 ? w.full_len[0] : w.full_len[1]);
}

// Key ranges (in key-tile units of `tile` keys) a training row group
// [q0, q0+R) must visit: up to two half-open tile ranges [t0, t1) and
// [t2, t3). Rows must lie in one half. Every live pair of the group lies in
// the union of the ranges (tiles may still hold dead pairs).
struct KeyRanges {
  int t0, t1, t2, t3;
};

BD3_HD KeyRanges train_key_ranges(int q0, int R, int n, int bs, int tile) {
  KeyRanges r;
  const bool qc = q0 >= n;
  const int r0 = qc ? q0 - n : q0;
  const int r1 = r0 + R - 1;
  const int b0 = r0 / bs, b1 = r1 / bs;
  if (!qc) {
    // own noisy blocks, then earlier clean blocks
    r.t0 = (bs * b0) / tile;
    r.t1 = (imin(bs * (b1 + 1), n) + tile - 1) / tile;
    r.t2 = n / tile;
    r.t3 = (n + bs * b1 + tile - 1) / tile;
  } else {
    r.t0 = n / tile;
    r.t1 = (n + imin(bs * (b1 + 1), n) + tile - 1) / tile;
    r.t2 = 0;
    r.t3 = 0;
  }
  return r;
}

// Query ranges (in query-tile units) that see a training key group
// [k0, k0+C) (keys in one half), the transpose of train_key_ranges: up to two
// half-open tile ranges. Used by the backward (one program per key tile).
BD3_HD KeyRanges train_query_ranges(int k0, int C, int n, int bs, int tile) {
  KeyRanges r;
  const bool kc = k0 >= n;
  const int a0 = kc ? k0 - n : k0;
  const int a1 = a0 + C - 1;
  const int kb0 = a0 / bs, kb1 = a1 / bs;
  if (!kc) {
    // noisy keys: noisy rows of the same blocks
    r.t0 = (bs * kb0) / tile;
    r.t1 = (imin(bs * (kb1 + 1), n) + tile - 1) / tile;
    r.t2 = 0;
    r.t3 = 0;
  } else {
    // clean keys of block kb: noisy rows of blocks > kb, clean rows of
    // blocks >= kb
    const int noisy_lo = imin(bs * (kb0 + 1), n);
    r.t0 = noisy_lo / tile;
    r.t1 = n / tile;
    if (r.t0 >= r.t1) { r.t0 = 0; r.t1 = 0; }
    r.t2 = (n + bs * kb0) / tile;
    r.t3 = (2 * n) / tile;
  }
  return r;
}

// Decode: classification of rows [i0, i0+R) (R >= 1, clamp to q_len done by
// the caller) against keys [j0, j0+C).
BD3_HD int decode_class(int i0, int R, int j0, int C, int q_len, int kv_len,
                        int bs) {
  const int i1 = imin(i0 + R, q_len) - 1;
  const int p0 = kv_len - q_len + i0, p1 = kv_len - q_len + i1;
  const int hi_first = imin((p0 / bs + 1) * bs, kv_len);  // row i0 sees [0, hi_first)
  const int hi_last = imin((p1 / bs + 1) * bs, kv_len);
  if (j0 >= hi_last) return kNone;
  if (j0 + C <= hi_first && i0 + R <= q_len) return kFull;
  return kPartial;
}

// Decode: one past the last key any row in [i0, i0+R) may see.
BD3_HD int decode_key_end(int i0, int R, int q_len, int kv_len, int bs) {
  const int i1 = imin(i0 + R, q_len) - 1;
  const int p1 = kv_len - q_len + i1;
  return imin((p1 / bs + 1) * bs, kv_len);
}

}  // namespace bd3
