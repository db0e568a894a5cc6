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
//   HBM once and kept in registers (d_model <= 4096).
// gate_residual_ln_modulate_kernel: the two fused (a residual update, then
//   the next sublayer's LayerNorm + modulate of the updated row).
// gate_residual_kernel: x + gate * y (the residual updates of
//   DiTBlock.forward, :560-566): gate * y in the promoted dtype of gate and y,
//   then the add in the promoted dtype of x and that product; bit-exact with
//   the eager ops. out may alias x.
#include "bd3_device.h"
#include "bd3_launch.h"

namespace bd3 {
namespace {

__device__ __forceinline__ float rbf(float f) { return (float)(__bf16)f; }  // round to bf16 (RNE)

// 8 consecutive elements starting at p (16-byte aligned for bf16, 32 for fp32).
__device__ __forceinline__ void load8(const void* p, int fp32, float (&v)[8]) {
  if (fp32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *(reinterpret_cast<const f32x4*>(p) + 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = a[k];
      v[4 + k] = b[k];
    }
  } else {
    const u32x4 w = ld16(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __builtin_bit_cast(float, w[k] << 16);
      v[2 * k + 1] = __builtin_bit_cast(float, w[k] & 0xffff0000u);
    }
  }
}

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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// LayerNorm statistics of a row held in registers (v: CH 16-byte chunks per
// lane, zero past the row), then modulate and store it. x_fp32: the row's
// dtype (the LayerNorm output is rounded back to it).
template <int CH>
__device__ __forceinline__ void ln_modulate_row(const GlueArgs& a, int b, int s, int lane,
                                                const float (&v)[CH][8], bool x_fp32) {
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
  const void* shr = elem(a.shift, a.m_fp32, b * a.sm_b);
  const void* scr = elem(a.scale, a.m_fp32, b * a.sm_b);
  void* outr = const_cast<char*>(elem(a.out, a.out_fp32, b * a.so_b + s * a.so_s));
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = lane + 64 * k;
    if (c >= nch) break;
    float w[8], sh[8], sc[8], o[8];
    load8(elem(a.weight, a.w_fp32, 8 * c), a.w_fp32, w);
    load8(elem(shr, a.m_fp32, 8 * c), a.m_fp32, sh);
    load8(elem(scr, a.m_fp32, 8 * c), a.m_fp32, sc);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float y = (w[e] * (v[k][e] - mean)) * inv;
      if (!x_fp32) y = rbf(y);  // .to(original dtype)
      // 1 + scale keeps scale's dtype (a Python scalar does not promote)
      const float t = a.m_fp32 ? 1.f + sc[e] : rbf(1.f + sc[e]);
      o[e] = mod_bf16 ? rbf(rbf(y * t) + sh[e]) : y * t + sh[e];
    }
    store8(static_cast<char*>(outr) + (int64_t)8 * c * (a.out_fp32 ? 4 : 2), a.out_fp32, o);
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
  const void* xr = elem(a.x, a.x_fp32, b * a.sx_b + s * a.sx_s);
  float v[CH][8];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = lane + 64 * k;
    if (c < nch) {
      load8(elem(xr, a.x_fp32, 8 * c), a.x_fp32, v[k]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[k][e] = 0.f;
    }
  }
  ln_modulate_row<CH>(a, b, s, lane, v, a.x_fp32);
}

// The residual update x + gate * y (gate_residual_kernel's dtypes and
// roundings) followed by modulate(LN(.)) of the updated row, which stays in
// registers: one launch and one read of the residual instead of two of each
// (DiTBlock.forward, model/modules.py:560-566 then the next sublayer's
// :537-568). out_x may alias x.
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
  const void* xr = elem(a.x, a.x_fp32, b * a.sx_b + s * a.sx_s);
  const void* gr = elem(a.gate, a.m_fp32, b * a.sm_b);
  const void* yr = elem(a.y, a.y_fp32, b * a.sy_b + s * a.sy_s);
  char* xo = const_cast<char*>(elem(a.out_x, !res_bf16, b * a.sxo_b + s * a.sxo_s));
  float v[CH][8];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int c = lane + 64 * k;
    if (c < nch) {
      float xv[8], gv[8], yv[8];
      load8(elem(xr, a.x_fp32, 8 * c), a.x_fp32, xv);
      load8(elem(gr, a.m_fp32, 8 * c), a.m_fp32, gv);
      load8(elem(yr, a.y_fp32, 8 * c), a.y_fp32, yv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float gy = gv[e] * yv[e];
        if (gy_bf16) gy = rbf(gy);
        const float o = xv[e] + gy;
        v[k][e] = res_bf16 ? rbf(o) : o;  // the value the residual store keeps
      }
      store8(xo + (int64_t)8 * c * (res_bf16 ? 2 : 4), !res_bf16, v[k]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[k][e] = 0.f;
    }
  }
  ln_modulate_row<CH>(a, b, s, lane, v, !res_bf16);
}

__global__ __launch_bounds__(256) void gate_residual_kernel(GlueArgs a) {
#pragma clang fp contract(off)  // gate * y rounded before the add, as the eager ops
  const int64_t e = (int64_t)wg_x() * 256 + wi_x();  // one 8-element chunk
  const int nch = a.d >> 3;
  if (e >= (int64_t)a.rows * nch) return;
  const int row = (int)(e / nch), c = (int)(e - (int64_t)row * nch);
  const int b = row / a.seq, s = row - b * a.seq;
  float x[8], g[8], y[8], o[8];
  load8(elem(a.x, a.x_fp32, b * a.sx_b + s * a.sx_s + 8 * c), a.x_fp32, x);
  load8(elem(a.shift, a.m_fp32, b * a.sm_b + 8 * c), a.m_fp32, g);  // gate
  load8(elem(a.y, a.y_fp32, b * a.sy_b + s * a.sy_s + 8 * c), a.y_fp32, y);
  const bool gy_bf16 = !a.m_fp32 && !a.y_fp32;
  const bool out_bf16 = !a.x_fp32 && gy_bf16;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float gy = g[k] * y[k];
    if (gy_bf16) gy = rbf(gy);
    o[k] = x[k] + gy;  // rounded to bf16 by the store when both are bf16
  }
  store8(const_cast<char*>(elem(a.out, !out_bf16, b * a.so_b + s * a.so_s + 8 * c)), !out_bf16, o);
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
  const int64_t n = (int64_t)a.rows * (a.d >> 3);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(gate_residual_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
