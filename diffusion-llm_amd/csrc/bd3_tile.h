// bd3_tile.h - shared pieces of the gfx950 training-attention kernels:
// cooperative 64-row tile staging (global -> VGPR -> padded LDS), transposed
// operand fetches, and the key/row interval masks written branch-free.
#pragma once

#include "bd3_device.h"
#include "bd3_mask.h"

namespace bd3 {

constexpr int kTileRows = 64;   // rows (keys or queries) per staged tile
constexpr int kLdsStride = 72;  // bf16 per LDS row: 64 + 8 pad (conflict-free b128 reads)
constexpr int kTileElems = kTileRows * kLdsStride;

// Stages 64-row x 64-col bf16 tiles of up to two tensors through VGPRs into
// padded LDS. Thread t moves 16-byte chunks c = t + j*THREADS: row c/8,
// column 8*(c%8), so 8 consecutive lanes read one 128-byte row.
template <int THREADS, int NT>
struct TileStager {
  static constexpr int kChunks = (kTileRows * 8) / THREADS;
  static_assert(kChunks * THREADS == kTileRows * 8, "threads must divide 512");
  u32x4 buf[NT][kChunks];
  int off[NT][kChunks];  // per-thread element offset of its chunk from the tile's row 0
  int lds_off[kChunks];

  __device__ __forceinline__ void init(int tid, const int64_t* row_stride) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * THREADS;
      lds_off[j] = (c >> 3) * kLdsStride + (c & 7) * 8;
#pragma unroll
      for (int t = 0; t < NT; ++t) off[t][j] = (c >> 3) * (int)row_stride[t] + (c & 7) * 8;
    }
  }
  // base[t] points at row 0 of the tile of tensor t.
  __device__ __forceinline__ void load(const uint16_t* const* base) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < kChunks; ++j) buf[t][j] = ld16(base[t] + off[t][j]);
  }
  __device__ __forceinline__ void store(__bf16* const* lds) const {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < kChunks; ++j) *reinterpret_cast<u32x4*>(lds[t] + lds_off[j]) = buf[t][j];
  }
};

// A/B operand of v_mfma_f32_32x32x16_bf16 taken from a row-major LDS tile in
// its natural layout: lane holds row (row0 + lane%32), columns
// 16c + 8*(lane/32) .. +7.
__device__ __forceinline__ bf16x8 lds_row_op(const __bf16* tile, int row0, int c, int lane) {
  return *reinterpret_cast<const bf16x8*>(
      &tile[(row0 + (lane & 31)) * kLdsStride + 16 * c + 8 * (lane >> 5)]);
}

// Transposed operand from a row-major LDS tile: lane receives column
// col0 + lane%32 and the 8 rows {r0 + 4g .. +3, r0 + 8 + 4g .. +3} with
// g = lane/32 (the row order of a 32x32 accumulator's register groups), via
// two ds_read_b64_tr_b16.
__device__ __forceinline__ bf16x8 lds_tr_op(const __bf16* tile, int r0, int col0, int lane) {
  const int row = r0 + 4 * (lane >> 5) + ((lane & 15) >> 2);
  const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  return cat8(lds_read_tr(&tile[row * kLdsStride + col]),
              lds_read_tr(&tile[(row + 8) * kLdsStride + col]));
}

// Group bounds for tile classification, moved to SGPRs once per wave so
// each per-tile classification is a few scalar compares.
__device__ __forceinline__ RowGroup uniform_row_group(int q0, int R, int n, int bs) {
  RowGroup g = train_row_group(q0, R, n, bs);
  g.clean = wave_uniform(g.clean);
  g.diag_lo = wave_uniform(g.diag_lo);
  g.diag_hi = wave_uniform(g.diag_hi);
  g.one_block = wave_uniform(g.one_block);
  g.full_end = wave_uniform(g.full_end);
  g.live_end = wave_uniform(g.live_end);
  return g;
}

__device__ __forceinline__ KeyGroup uniform_key_group(int k0, int C, int n, int bs) {
  KeyGroup g = train_key_group(k0, C, n, bs);
  g.clean = wave_uniform(g.clean);
  g.noisy_lo = wave_uniform(g.noisy_lo);
  g.noisy_hi = wave_uniform(g.noisy_hi);
  g.one_block = wave_uniform(g.one_block);
  g.nz_live_lo = wave_uniform(g.nz_live_lo);
  g.nz_full_lo = wave_uniform(g.nz_full_lo);
  g.cl_live_lo = wave_uniform(g.cl_live_lo);
  g.cl_full_lo = wave_uniform(g.cl_full_lo);
  return g;
}

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

// Sum of the 8 bf16 values of a P operand added to acc, as 4 v_dot2c_f32_bf16
// against (1, 1): the softmax denominator accumulates exactly the rounded
// probabilities the PV product uses, at half the VALU cost of fp32 adds.
__device__ __forceinline__ float sum_bf16x8(bf16x8 v, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), one, acc, false);
  return acc;
}

// Visibility of key k for a row with intervals iv, as 0/1 without branches.
__device__ __forceinline__ bool iv_has(const RowIntervals& iv, int k) {
  return ((unsigned)(k - iv.lo1) < (unsigned)(iv.hi1 - iv.lo1)) |
         ((unsigned)(k - iv.lo2) < (unsigned)(iv.hi2 - iv.lo2));
}

// Work order shared by the training kernels: blockIdx.x -> (rank, bh) with
// bh fastest, so that every tile of one (b, h) lands on the same XCD when
// bh % 8 == 0 (workgroups are dealt to the 8 XCDs round-robin); rank 0 is the
// heaviest tile.
struct BlockOrder {
  int rank, bh, b, h;
  __device__ __forceinline__ BlockOrder(int bhs, int heads) {
    rank = blockIdx.x / bhs;
    bh = blockIdx.x - rank * bhs;
    b = bh / heads;
    h = bh - b * heads;
  }
};

}  // namespace bd3
