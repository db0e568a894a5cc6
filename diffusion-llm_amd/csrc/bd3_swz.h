// bd3_swz.h - swizzled 64x64 bf16 tiles in LDS, filled by direct
// global -> LDS loads (global_load_lds_dwordx4, gfx950), and the operand
// fetches of v_mfma_f32_32x32x16_bf16 from them.
//
// Layout: a tile is 64 rows of 64 bf16 (128-byte rows, no padding). The
// 16-byte chunk c (columns 8c .. 8c+7) of row r is stored at chunk position
// c ^ swz(r), swz(r) = ((r & 2) << 1) | ((r >> 2) & 3) (row bits 1..3). The
// LDS has 64 four-byte banks (256 bytes per cycle); the swizzle keeps both
// read patterns free of bank conflicts (measured on MI355X):
//   * row operands (ds_read_b128, 16 lanes per cycle): 16 consecutive rows,
//     same logical chunk. Even rows share one half of the 256-byte window,
//     odd rows the other; swz is a bijection of (r >> 1) & 7, so the 8 rows
//     of each parity land on 8 distinct 16-byte slots;
//   * transposed operands (ds_read_b64_tr_b16, 32 lanes per cycle): rows
//     r0 .. r0+3 (r0 % 4 == 0) x 4 adjacent chunks of one aligned group of 4.
//     Rows r0 and r0+2 (one parity) differ in bit 2 of swz, so their chunks
//     fall in different aligned groups of 4 positions: 16 distinct slots.
//
// Direct loads: one wave instruction writes 64 lanes x 16 bytes = one 1 KB
// block (8 rows) contiguously at the wave-uniform LDS base (M0); lane L lands
// at chunk position L % 8 of row 8b + L / 8 of block b, so it fetches logical
// chunk (L % 8) ^ swz(8b + L / 8) of that row from global memory.
#pragma once

#include "bd3_device.h"

namespace bd3 {

constexpr int kSwRows = 64;
constexpr int kSwTile = kSwRows * 64;  // bf16 elements per tile (8 KB)

__device__ __forceinline__ int swz(int r) { return ((r & 2) << 1) | ((r >> 2) & 3); }

typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte direct load per lane into the 1 KB LDS block at byte address
// `lds_addr` (global_load_lds_dwordx4 with that address in M0): lane L reads
// the 16 bytes at base + off_bytes (its own 32-bit offset from the
// wave-uniform base) and writes them to lds_addr + 16 L.
//
// Issued as inline assembly on purpose: the compiler cannot tell the ring
// stages apart, so with the builtin it waits for every outstanding direct
// load (vmcnt(0)) before the next LDS read of any stage, which serialises the
// prefetch. The kernels instead wait explicitly (a counted vmcnt) before the
// barrier that publishes a stage. The compiler never keeps
// a value in M0 across statements on this path (it sets M0 right before each
// of its own uses), so clobbering it here is safe.
__device__ __forceinline__ void dma16(const void* base, uint32_t off_bytes, uint32_t lds_addr) {
  const uint64_t sb = (uint64_t)(uintptr_t)uniform_ptr(base);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(wave_uniform_u32(lds_addr)), "v"(off_bytes), "s"(sb)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// The same with a per-lane 64-bit global address (lanes may read from
// different buffers).
__device__ __forceinline__ void dma16_va(const void* addr, uint32_t lds_addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(wave_uniform_u32(lds_addr)), "v"(addr)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return wave_uniform_u32((uint32_t)(uintptr_t)((const lds_void*)p));
}

// Waits until at most N of this wave's vector-memory loads are outstanding
// (direct loads retire in issue order), then joins the workgroup barrier.
// Both are in one asm statement with a memory clobber, so the compiler moves
// no LDS access across the barrier and adds no vmcnt(0) of its own (its
// __syncthreads would wait for every direct load still in flight).
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Row operand (A or B of a 32x32x16 MFMA whose k index runs along the tile's
// columns): lane holds row row0 + lane%32, columns 16c + 8*(lane/32) .. +7.
// row0 must be a multiple of 16.
__device__ __forceinline__ bf16x8 sw_row_op(const __bf16* tile, int row0, int c, int lane) {
  const int r = lane & 31;
  const int chunk = (2 * c + (lane >> 5)) ^ swz(r);
  return *reinterpret_cast<const bf16x8*>(&tile[(row0 + r) * 64 + chunk * 8]);
}

// Transposed operand: lane receives column col0 + lane%32 and the 8 rows
// {r0 + 4g .. +3, r0 + 8 + 4g .. +3}, g = lane/32 (the row order of a 32x32
// accumulator's register groups), via two ds_read_b64_tr_b16. r0 multiple
// of 16, col0 multiple of 16.
__device__ __forceinline__ bf16x8 sw_tr_op(const __bf16* tile, int r0, int col0, int lane) {
  const int rr = 4 * (lane >> 5) + ((lane & 15) >> 2);  // row offset, < 8
  const int col = col0 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int off0 = (r0 + rr) * 64 + (((col >> 3) ^ swz(rr)) << 3) + (col & 7);
  const int off1 = (r0 + rr + 8) * 64 + (((col >> 3) ^ swz(rr + 8)) << 3) + (col & 7);
  return cat8(lds_read_tr(&tile[off0]), lds_read_tr(&tile[off1]));
}

}  // namespace bd3
