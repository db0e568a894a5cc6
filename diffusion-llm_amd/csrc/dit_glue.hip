// dit_glue.hip - the elementwise work around attention in a DiT block, fused.
//
// ln_modulate_kernel: modulate(LN(x), shift, scale) of DiTBlock.forward
//   (model/modules.py:537-568) with the weight-only LayerNorm
//   (model/modules.py:243-288) and modulate (model/modules.py:778-788), one
//   read of x and one write of the result instead of ~8 eager ops:
//     mean, var (correction 0) of the fp32-upcast row; inv = rsqrt(var + eps);
//     y = (w * (x - mean)) * inv in fp32, cast back to x's dtype;
//     out = y * (1 + scale) + shift: 1 + scale in the vectors' dtype (a
//     Python scalar does not promote), the product and the sum in the
//     promoted dtype of y and the vectors (bf16 if both are bf16, every op
//     rounded, as eager bf16 tensor ops; fp32 otherwise), optionally rounded
//     to bf16 for the next matmul (what autocast does at its input).
//   One wavefront per row (64 lanes x 16-byte chunks); the row is read from
//   HBM once and kept in registers (d_model <= 4096). Every load of a row and
//   of its vectors is issued before the first use (loads whose dtype is a
//   run-time flag are issued as raw 16-byte pairs and decoded later, so no
//   branch separates them), and the row sums are reduced with DPP and
//   permlane swaps instead of LDS permutes.
// gate_residual_ln_modulate_kernel: the two fused (a residual update, then
//   the next sublayer's LayerNorm + modulate of the updated row).
// gate_residual_kernel: x + gate * y (the residual updates of
//   DiTBlock.forward, :560-566): gate * y in the promoted dtype of gate and y,
//   then the add in the promoted dtype of x and that product; bit-exact with
//   the eager ops. out may alias x.
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"

namespace bd3 {
namespace {

__device__ __forceinline__ float rbf(float f) { return (float)(__bf16)f; }  // round to bf16 (RNE)

// 8 consecutive elements starting at p (16-byte aligned for bf16, 32 for
// fp32) as raw bits: two 16-byte loads, the second of the same 16 bytes when
// the elements are bf16, so the pair is issued without a branch on the dtype.
struct Raw8 {
  u32x4 lo, hi;
};

__device__ __forceinline__ Raw8 ld_raw8(const void* p, int fp32) {
  Raw8 r;
  r.lo = ld16(p);
  r.hi = ld16(static_cast<const char*>(p) + (fp32 ? 16 : 0));
  return r;
}

__device__ __forceinline__ void unpack8(const Raw8& r, int fp32, float (&v)[8]) {
  float f[8], b[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    // (element values first: __builtin_bit_cast of a vector element lvalue
    // reads element 0 with this compiler)
    const uint32_t l = r.lo[k], h = r.hi[k];
    f[k] = __uint_as_float(l);
    f[4 + k] = __uint_as_float(h);
    b[2 * k] = __uint_as_float(l << 16);
    b[2 * k + 1] = __uint_as_float(l & 0xffff0000u);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = fp32 ? f[e] : b[e];
}

__device__ __forceinline__ void load8(const void* p, int fp32, float (&v)[8]) { unpack8(ld_raw8(p, fp32), fp32, v); }

__device__ __forceinline__ void store8(void* p, int fp32, const float (&v)[8]) {
  if (fp32) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *(reinterpret_cast<f32x4*>(p) + 1) = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    *reinterpret_cast<bf16x8*>(p) = to_bf16x8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
  }
}

__device__ __forceinline__ const char* elem(const void* base, int fp32, int64_t i) {
  return static_cast<const char*>(base) + i * (fp32 ? 4 : 2);
}

__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
  int t;
  switch (ctrl_sel) {
    case 0: t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad [1,0,3,2]
    case 1: t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad [2,3,0,1]
    case 2: t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false); break; // row_mirror
  }
  return v + __int_as_float(t);
}

// Sum over the 64 lanes, the total in every lane: lane pairs i ^ 1, i ^ 2
// (quad permutes), then the mirrored lane within 8 and within 16 (each lane
// of a quad / half-row holds the same partial by then, so the mirror pairs
// the same partials as i ^ 4, i ^ 8), then rows i ^ 16 and halves i ^ 32
// (permlane swaps).
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add(v, 0);
  v = dpp_add(v, 1);
  v = dpp_add(v, 2);
  v = dpp_add(v, 3);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// The LayerNorm weight and the shift / scale of one row's batch index, as
// raw loads: for rows of up to CH = 4 chunks per lane all of them are issued
// with the row's own loads (PRE); longer rows load each chunk's vectors where
// they are used (registers go to the row).
template <int CH, bool PRE = (CH <= 4)>
struct ModVecs {
  Raw8 w[PRE ? CH : 1], sh[PRE ? CH : 1], sc[PRE ? CH : 1];
  const char* shr;
  const char* scr;
  __device__ __forceinline__ ModVecs(const GlueArgs& a, int b, int lane) {
    shr = elem(a.shift, a.m_fp32, (int64_t)b * a.sm_b);
    scr = elem(a.scale, a.m_fp32, (int64_t)b * a.sm_b);
    if constexpr (PRE) {
      const int nch = a.d >> 3;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int c = imin(lane + 64 * k, nch - 1);  // lanes past the row repeat its last chunk
        w[k] = ld_raw8(elem(a.weight, a.w_fp32, 8 * c), a.w_fp32);
        sh[k] = ld_raw8(elem(shr, a.m_fp32, 8 * c), a.m_fp32);
        sc[k] = ld_raw8(elem(scr, a.m_fp32, 8 * c), a.m_fp32);
      }
    }
  }
  __device__ __forceinline__ void chunk(const GlueArgs& a, int k, int c, float (&w8)[8], float (&sh8)[8],
                                        float (&sc8)[8]) const {
    if constexpr (PRE) {
      unpack8(w[k], a.w_fp32, w8);
      unpack8(sh[k], a.m_fp32, sh8);
      unpack8(sc[k], a.m_fp32, sc8);
    } else {
      load8(elem(a.weight, a.w_fp32, 8 * c), a.w_fp32, w8);
      load8(elem(shr, a.m_fp32, 8 * c), a.m_fp32, sh8);
      load8(elem(scr, a.m_fp32, 8 * c), a.m_fp32, sc8);
    }
  }
};

// LayerNorm statistics of a row held in registers (v: CH 16-byte chunks per
// lane, zero past the row), then modulate with the row's vectors and store
// it. x_fp32: the row's dtype (the LayerNorm output is rounded back to it).
template <int CH, class MV>
__device__ __forceinline__ void ln_modulate_row(const GlueArgs& a, int b, int s, int lane,
                                                const float (&v)[CH][8], const MV& mv, bool x_fp32) {
#pragma clang fp contract(off)  // separate products and sums, as the eager ops
  const int D = a.d;
  const int nch = D >> 3;
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += v[k][e];
  const float mean = wave_sum(sum) / (float)D;
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < CH; ++k)
    if (lane + 64 * k < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dlt = v[k][e] - mean;
        sq += dlt * dlt;
      }
    }
  const float inv = rsqrtf(wave_sum(sq) / (float)D + a.eps);

  const bool mod_bf16 = !x_fp32 && !a.m_fp32;  // modulate in bf16 iff y and the vectors are bf16
  char* outr = const_cast<char*>(elem(a.out, a.out_fp32, (int64_t)b * a.so_b + (int64_t)s * a.so_s));
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = lane + 64 * k;
    if (c >= nch) break;
    float w[8], sh[8], sc[8], o[8];
    mv.chunk(a, k, c, w, sh, sc);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float y = (w[e] * (v[k][e] - mean)) * inv;
      if (!x_fp32) y = rbf(y);  // .to(original dtype)
      // 1 + scale keeps scale's dtype (a Python scalar does not promote)
      const float t = a.m_fp32 ? 1.f + sc[e] : rbf(1.f + sc[e]);
      o[e] = mod_bf16 ? rbf(rbf(y * t) + sh[e]) : y * t + sh[e];
    }
    store8(outr + (int64_t)8 * c * (a.out_fp32 ? 4 : 2), a.out_fp32, o);
  }
}

// Chunk k of a lane, zero past the row.
template <int CH>
__device__ __forceinline__ void unpack_row(const Raw8 (&r)[CH], int fp32, int lane, int nch, float (&v)[CH][8]) {
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    unpack8(r[k], fp32, v[k]);
    const bool in = lane + 64 * k < nch;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[k][e] = in ? v[k][e] : 0.f;
  }
}

// CH: 16-byte chunks (8 elements) of the row held per lane; the row is read
// from HBM once into registers (d_model <= 512 * CH).
template <int CH>
__global__ __launch_bounds__(256) void ln_modulate_kernel(GlueArgs a) {
  const int row = wg_x() * 4 + (wi_x() >> 6);
  if (row >= a.rows) return;
  const int lane = wi_x() & 63;
  const int b = row / a.seq, s = row - b * a.seq;
  const int nch = a.d >> 3;
  const void* xr = elem(a.x, a.x_fp32, (int64_t)b * a.sx_b + (int64_t)s * a.sx_s);
  Raw8 xraw[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) xraw[k] = ld_raw8(elem(xr, a.x_fp32, 8 * imin(lane + 64 * k, nch - 1)), a.x_fp32);
  const ModVecs<CH> mv(a, b, lane);
  float v[CH][8];
  unpack_row<CH>(xraw, a.x_fp32, lane, nch, v);
  ln_modulate_row<CH>(a, b, s, lane, v, mv, a.x_fp32);
}

// The residual update x + gate * y (gate_residual_kernel's dtypes and
// roundings) followed by modulate(LN(.)) of the updated row, which stays in
// registers: one launch and one read of the residual instead of two of each
// (DiTBlock.forward, model/modules.py:560-566 then the next sublayer's
// :537-568). out_x may alias x (each lane reads its chunks before it writes
// them).
template <int CH>
__global__ __launch_bounds__(256) void gate_residual_ln_modulate_kernel(GlueArgs a) {
#pragma clang fp contract(off)  // gate * y rounded before the add, as the eager ops
  const int row = wg_x() * 4 + (wi_x() >> 6);
  if (row >= a.rows) return;
  const int lane = wi_x() & 63;
  const int b = row / a.seq, s = row - b * a.seq;
  const int nch = a.d >> 3;
  const bool gy_bf16 = !a.m_fp32 && !a.y_fp32;
  const bool res_bf16 = !a.x_fp32 && gy_bf16;  // dtype of x + gate * y
  const void* xr = elem(a.x, a.x_fp32, (int64_t)b * a.sx_b + (int64_t)s * a.sx_s);
  const void* gr = elem(a.gate, a.m_fp32, (int64_t)b * a.sm_b);
  const void* yr = elem(a.y, a.y_fp32, (int64_t)b * a.sy_b + (int64_t)s * a.sy_s);
  char* xo = const_cast<char*>(elem(a.out_x, !res_bf16, (int64_t)b * a.sxo_b + (int64_t)s * a.sxo_s));
  Raw8 xraw[CH], graw[CH], yraw[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = imin(lane + 64 * k, nch - 1);
    xraw[k] = ld_raw8(elem(xr, a.x_fp32, 8 * c), a.x_fp32);
    graw[k] = ld_raw8(elem(gr, a.m_fp32, 8 * c), a.m_fp32);
    yraw[k] = ld_raw8(elem(yr, a.y_fp32, 8 * c), a.y_fp32);
  }
  const ModVecs<CH> mv(a, b, lane);
  float v[CH][8];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = lane + 64 * k;
    float xv[8], gv[8], yv[8];
    unpack8(xraw[k], a.x_fp32, xv);
    unpack8(graw[k], a.m_fp32, gv);
    unpack8(yraw[k], a.y_fp32, yv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float gy = gv[e] * yv[e];
      if (gy_bf16) gy = rbf(gy);
      const float o = xv[e] + gy;
      v[k][e] = c < nch ? (res_bf16 ? rbf(o) : o) : 0.f;  // the value the residual store keeps
    }
    if (c < nch) store8(xo + (int64_t)8 * c * (res_bf16 ? 2 : 4), !res_bf16, v[k]);
  }
  ln_modulate_row<CH>(a, b, s, lane, v, mv, !res_bf16);
}

// 4 consecutive elements at p: fp32 (16 bytes) or bf16 (8 bytes), the dtype
// fixed at compile time.
template <bool F32>
__device__ __forceinline__ void load4(const void* p, float (&v)[4]) {
  if constexpr (F32) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = t[k];
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(t.x << 16);
    v[1] = __uint_as_float(t.x & 0xffff0000u);
    v[2] = __uint_as_float(t.y << 16);
    v[3] = __uint_as_float(t.y & 0xffff0000u);
  }
}

// x + gate * y with an fp32 residual (the result is fp32): 4 elements per
// thread, so each load of x (16 bytes per lane) covers one contiguous 1 KB
// per wave, where 8-element chunks (two 16-byte halves 32 bytes apart per
// lane) split every load across twice the span. GF / YF: gate / y in fp32.
// Measured at 8 x 2048 x 768: 25.8 -> 23.3 us, bit-identical.
template <bool GF, bool YF>
__global__ __launch_bounds__(256) void gate_residual_f32_kernel(GlueArgs a) {
#pragma clang fp contract(off)  // gate * y rounded before the add, as the eager ops
  const int64_t e = (int64_t)wg_x() * 256 + wi_x();  // one 4-element chunk
  const int nch = a.d >> 2;
  if (e >= (int64_t)a.rows * nch) return;
  const int row = (int)(e / nch), c = (int)(e - (int64_t)row * nch);
  const int b = row / a.seq, s = row - b * a.seq;
  float x[4], g[4], y[4];
  load4<true>(static_cast<const float*>(a.x) + (int64_t)b * a.sx_b + (int64_t)s * a.sx_s + 4 * c, x);
  load4<GF>(elem(a.shift, GF, (int64_t)b * a.sm_b + 4 * c), g);  // gate
  load4<YF>(elem(a.y, YF, (int64_t)b * a.sy_b + (int64_t)s * a.sy_s + 4 * c), y);
  const bool gy_bf16 = !GF && !YF;
  f32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float gy = g[k] * y[k];
    if (gy_bf16) gy = rbf(gy);
    o[k] = x[k] + gy;
  }
  *reinterpret_cast<f32x4*>(static_cast<float*>(a.out) + (int64_t)b * a.so_b + (int64_t)s * a.so_s + 4 * c) = o;
}

__global__ __launch_bounds__(256) void gate_residual_kernel(GlueArgs a) {
#pragma clang fp contract(off)  // gate * y rounded before the add, as the eager ops
  const int64_t e = (int64_t)wg_x() * 256 + wi_x();  // one 8-element chunk
  const int nch = a.d >> 3;
  if (e >= (int64_t)a.rows * nch) return;
  const int row = (int)(e / nch), c = (int)(e - (int64_t)row * nch);
  const int b = row / a.seq, s = row - b * a.seq;
  const Raw8 xr = ld_raw8(elem(a.x, a.x_fp32, (int64_t)b * a.sx_b + (int64_t)s * a.sx_s + 8 * c), a.x_fp32);
  const Raw8 gr = ld_raw8(elem(a.shift, a.m_fp32, (int64_t)b * a.sm_b + 8 * c), a.m_fp32);  // gate
  const Raw8 yr = ld_raw8(elem(a.y, a.y_fp32, (int64_t)b * a.sy_b + (int64_t)s * a.sy_s + 8 * c), a.y_fp32);
  float x[8], g[8], y[8], o[8];
  unpack8(xr, a.x_fp32, x);
  unpack8(gr, a.m_fp32, g);
  unpack8(yr, a.y_fp32, y);
  const bool gy_bf16 = !a.m_fp32 && !a.y_fp32;
  const bool out_bf16 = !a.x_fp32 && gy_bf16;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float gy = g[k] * y[k];
    if (gy_bf16) gy = rbf(gy);
    o[k] = x[k] + gy;  // rounded to bf16 by the store when both are bf16
  }
  store8(const_cast<char*>(elem(a.out, !out_bf16, (int64_t)b * a.so_b + (int64_t)s * a.so_s + 8 * c)), !out_bf16, o);
}

}  // namespace

hipError_t launch_ln_modulate(const GlueArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  const int ch = (a.d / 8 + 63) / 64;  // chunks per lane
  if (ch <= 1)
    hipLaunchKernelGGL(ln_modulate_kernel<1>, grid, dim3(256), 0, stream, a);
  else if (ch <= 2)
    hipLaunchKernelGGL(ln_modulate_kernel<2>, grid, dim3(256), 0, stream, a);
  else if (ch <= 4)
    hipLaunchKernelGGL(ln_modulate_kernel<4>, grid, dim3(256), 0, stream, a);
  else if (ch <= 8)
    hipLaunchKernelGGL(ln_modulate_kernel<8>, grid, dim3(256), 0, stream, a);
  else
    return hipErrorInvalidValue;  // d_model > 4096: rejected by the C ABI
  return hipGetLastError();
}

hipError_t launch_gate_residual_ln_modulate(const GlueArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  const int ch = (a.d / 8 + 63) / 64;  // chunks per lane
  if (ch <= 1)
    hipLaunchKernelGGL(gate_residual_ln_modulate_kernel<1>, grid, dim3(256), 0, stream, a);
  else if (ch <= 2)
    hipLaunchKernelGGL(gate_residual_ln_modulate_kernel<2>, grid, dim3(256), 0, stream, a);
  else if (ch <= 4)
    hipLaunchKernelGGL(gate_residual_ln_modulate_kernel<4>, grid, dim3(256), 0, stream, a);
  else if (ch <= 8)
    hipLaunchKernelGGL(gate_residual_ln_modulate_kernel<8>, grid, dim3(256), 0, stream, a);
  else
    return hipErrorInvalidValue;  // d_model > 4096: rejected by the C ABI
  return hipGetLastError();
}

hipError_t launch_gate_residual(const GlueArgs& a, hipStream_t stream) {
  if (a.x_fp32) {  // fp32 residual and result: 4-element chunks
    const int64_t n4 = (int64_t)a.rows * (a.d >> 2);
    if (n4 == 0) return hipSuccess;
    const dim3 grid((unsigned)((n4 + 255) / 256));
    if (a.m_fp32 && a.y_fp32)
      hipLaunchKernelGGL((gate_residual_f32_kernel<true, true>), grid, dim3(256), 0, stream, a);
    else if (a.m_fp32)
      hipLaunchKernelGGL((gate_residual_f32_kernel<true, false>), grid, dim3(256), 0, stream, a);
    else if (a.y_fp32)
      hipLaunchKernelGGL((gate_residual_f32_kernel<false, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((gate_residual_f32_kernel<false, false>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  const int64_t n = (int64_t)a.rows * (a.d >> 3);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(gate_residual_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
