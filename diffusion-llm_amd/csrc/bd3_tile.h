// bd3_tile.h - shared pieces of the gfx950 training-attention kernels: the
// padded LDS layout of the dK/dV epilogue, class thresholds in SGPRs, the
// bf16 row sums, the branch-free interval mask test and the workgroup order.
#pragma once

#include "bd3_device.h"
#include "bd3_mask.h"

namespace bd3 {

constexpr int kLdsStride = 72;  // bf16 per padded LDS row: 64 + 8 pad (conflict-free b128 reads)
constexpr int kTileElems = 64 * kLdsStride;  // one 64-row padded tile

// Class thresholds moved to SGPRs (they are the same for the whole wave).
__device__ __forceinline__ ClassBounds uniform_bounds(ClassBounds b) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    b.lo[h] = wave_uniform(b.lo[h]);
    b.hi[h] = wave_uniform(b.hi[h]);
    b.flo[h] = wave_uniform(b.flo[h]);
    b.fhi[h] = wave_uniform(b.fhi[h]);
  }
  return b;
}

// Walk-index class intervals moved to SGPRs.
__device__ __forceinline__ WalkClasses uniform_walk(WalkClasses w) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    w.live_lo[r] = wave_uniform(w.live_lo[r]);
    w.live_len[r] = wave_uniform(w.live_len[r]);
    w.full_lo[r] = wave_uniform(w.full_lo[r]);
    w.full_len[r] = wave_uniform(w.full_len[r]);
  }
  return w;
}

// Visibility of key k for a row with intervals iv, as 0/1 without branches.
__device__ __forceinline__ bool iv_has(const RowIntervals& iv, int k) {
  return ((unsigned)(k - iv.lo1) < (unsigned)(iv.hi1 - iv.lo1)) |
         ((unsigned)(k - iv.lo2) < (unsigned)(iv.hi2 - iv.lo2));
}

// Work order shared by the training kernels: workgroup id -> (rank, bh) with
// bh fastest, so that every tile of one (b, h) lands on the same XCD when
// bh % 8 == 0 (workgroups are dealt to the 8 XCDs round-robin); rank 0 is the
// heaviest tile.
struct BlockOrder {
  int rank, bh, b, h;
  __device__ __forceinline__ BlockOrder(int bhs, int heads) : BlockOrder(wg_x(), bhs, heads) {}
  __device__ __forceinline__ BlockOrder(int id, int bhs, int heads) {
    rank = id / bhs;
    bh = id - rank * bhs;
    b = bh / heads;
    h = bh - b * heads;
  }
};

// The tiles a workgroup visits are t0 .. t0 + n_first - 1, then t2, t2 + 1,
// ... (the two live ranges of the schedule; the first may be empty). TileWalk yields, one call per
// tile, the index and a byte offset scaled by a per-tile stride, by
// increments instead of a 64-bit multiply per tile (all wave-uniform).
struct TileWalk {
  int tile, left, t2;
  __device__ __forceinline__ TileWalk(int t0_, int n_first, int t2_)
      : tile(n_first > 0 ? t0_ : t2_), left(n_first), t2(t2_) {}
  __device__ __forceinline__ void next() {
    --left;
    tile = left == 0 ? t2 : tile + 1;
  }
};

// A wave-uniform pointer moving along such a walk: `step` bytes per tile,
// jumping to the second range's first tile when the first range ends.
struct TilePtr {
  const char* cur;
  const char* jump;
  int64_t step;
  __device__ __forceinline__ TilePtr(const void* base, int64_t step_bytes, int t0, int n_first, int t2)
      : cur(static_cast<const char*>(base) + (int64_t)(n_first > 0 ? t0 : t2) * step_bytes),
        jump(static_cast<const char*>(base) + (int64_t)t2 * step_bytes),
        step(step_bytes) {}
  // `jumping`: this step leaves the first range
  __device__ __forceinline__ void next(bool jumping) { cur = jumping ? jump : cur + step; }
};

}  // namespace bd3
