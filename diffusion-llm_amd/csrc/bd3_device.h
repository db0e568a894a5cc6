// bd3_device.h - gfx950 (CDNA4) building blocks for the BD3-LM attention
// kernels: MFMA wrappers, LDS transpose reads, bf16 packing, fast exp2.
//
// Lane layouts (wave64, verified on MI355X with an in-bounds probe):
//   v_mfma_f32_32x32x16_bf16  D(32x32) += A(32x16) * B(16x32)
//     A[i][k]: lane i%32 + 32*(k/8), element k%8 of the lane's 8 bf16
//     B[k][j]: lane j%32 + 32*(k/8), element k%8
//     D[i][j]: lane j + 32*((i/4)%2), register (i/8)*4 + i%4
//   v_mfma_f32_16x16x32_bf16  D(16x16) += A(16x32) * B(32x16)
//     A[i][k]: lane i + 16*(k/8), element k%8;  B[k][j]: lane j + 16*(k/8)
//     D[i][j]: lane j + 16*(i/4), register i%4
//   ds_read_b64_tr_b16 (per 16-lane group, each lane supplies an 8-byte
//     address): result lane i, element j = element i%4 of the chunk that
//     source lane 4*j + i/4 addressed. If source lane s addresses row
//     (r0 + s/4), columns (c0 + 4*(s%4) .. +3) of a row-major matrix, lane i
//     receives column c0 + i, rows r0 .. r0+3: a transposed 4x16 tile.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bd3_launch.h"

namespace bd3 {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Transposed LDS read (see the layout note above).
__device__ __forceinline__ bf16x4 lds_read_tr(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Round-to-nearest-even fp32 -> bf16 of 8 values (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 to_bf16x8(float a0, float a1, float a2,
                                            float a3, float a4, float a5,
                                            float a6, float a7) {
  bf16x8 r = {(__bf16)a0, (__bf16)a1, (__bf16)a2, (__bf16)a3,
              (__bf16)a4, (__bf16)a5, (__bf16)a6, (__bf16)a7};
  return r;
}

__device__ __forceinline__ bf16x4 to_bf16x4(float a0, float a1, float a2,
                                            float a3) {
  bf16x4 r = {(__bf16)a0, (__bf16)a1, (__bf16)a2, (__bf16)a3};
  return r;
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float fast_log2(float x) {
  return __builtin_amdgcn_logf(x);
}

// v_permlane32_swap(vdst = x, src0 = x) leaves {x_own, x_partner} in the two
// results, in an order that depends on the lane half (lanes 0-31 keep vdst
// and receive the upper half's value in src0; lanes 32-63 the reverse), so a
// symmetric combine of both results needs no select.
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                            __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                            __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float shfl_xor(float x, int m) {
  return __shfl_xor(x, m, 64);
}

// Work-item and workgroup ids read from the hardware-initialised registers.
// threadIdx / blockIdx go through calls to the device library's
// __ockl_get_local_id / __ockl_get_group_id, which this toolchain leaves out
// of line at -O3 (an s_swappc and the call ABI's register conventions in
// every kernel prologue).
__device__ __forceinline__ int wi_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int wg_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int wg_y() { return (int)__builtin_amdgcn_workgroup_id_y(); }
__device__ __forceinline__ int wg_z() { return (int)__builtin_amdgcn_workgroup_id_z(); }

// A value the program knows to be the same in every lane of the wave (the
// wave index, tile counts derived from blockIdx): moving it to an SGPR lets
// the compiler branch on it with scalar branches instead of exec masks.
__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint32_t wave_uniform_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}
// A wave-uniform pointer moved to SGPRs, so address arithmetic on it stays
// scalar. readfirstlane returns int: each half goes through uint32_t so the
// low half is zero-extended (a sign-extended low half would corrupt the high).
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t b = (uint64_t)(uintptr_t)p;
  const uint64_t u = (uint64_t)wave_uniform_u32((uint32_t)b) | ((uint64_t)wave_uniform_u32((uint32_t)(b >> 32)) << 32);
  return (T*)(uintptr_t)u;
}


// 16-byte global load/store helpers (bf16 rows are 128 B at head_dim 64).
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Non-temporal 16-byte load: for data read exactly once (the decode KV stream).
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

}  // namespace bd3
