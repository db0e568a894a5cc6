// qkv_rope.hip - the attention inputs of one BD3-LM layer, written where the
// attention reads them.
//
// qkv_rope_kernel: counterpart of the head split, the two RoPE calls and the
//   cache concatenation of BidirectionalMultiHeadAttention.forward
//   (model/modules.py:395-414) with RoPE.forward (model/modules.py:212-240).
//   One pass over the fused projection (batch, seq, 3 * heads * 64): q and k
//   are rotated and stored, v is copied, each to its own (b, h, s)-strided
//   destination, which may be a slot of a preallocated KV cache. The rotation
//   repeats the reference's eager bf16 arithmetic step by step, so the result
//   is bit-identical to it: the fp32 sin / cos table rows are rounded to bf16
//   (`.to(x.dtype)`), and each of x1*cos, x2*sin, x1*sin, x2*cos, the
//   difference and the sum is rounded to bf16 (round to nearest even) as a
//   separate bf16 tensor op would. A product of two bf16 values is exact in
//   fp32, so only these roundings matter.
//
// kv_write_kernel: the strided copy of KVCache.append (model/kv_cache.py:42-55)
//   into a preallocated cache slot instead of a torch.cat reallocation.
#include "bd3_device.h"
#include "bd3_launch.h"

namespace bd3 {
namespace {

// Rounding to bf16 uses the hardware conversion (v_cvt_pk_bf16_f32, round to
// nearest even). Measured on MI355X against the bit-level definition over
// normal, subnormal (including subnormal products), zero, infinite and
// boundary values, it differs only for NaN, whose sign and payload it keeps;
// torch returns the canonical 0x7fc0 for every NaN. A NaN anywhere in the
// chain makes the final result NaN, so only the stored values are
// canonicalised.
// One instruction for both values: written as inline assembly because the
// compiler otherwise converts each value on its own and re-packs them with
// shifts and masks when the packed result is unpacked again.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
  return r;
}
__device__ __forceinline__ float lo_f(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Every NaN half of a packed pair -> 0x7fc0. A half h is NaN iff
// (h & 0x7fff) > 0x7f80, i.e. (h & 0x7fff) + 0x7f carries into bit 15.
__device__ __forceinline__ uint32_t canon_nan(uint32_t w) {
  const uint32_t t = ((w & 0x7fff7fffu) + 0x007f007fu) & 0x80008000u;
  const uint32_t m = (t >> 15) * 0xffffu;  // 0xffff in each NaN half
  return (w & ~m) | (0x7fc07fc0u & m);
}

// Rotates the 8 coordinate pairs (8j + i, 32 + 8j + i), i = 0..7, of one
// head row held as two 16-byte halves x1 (coordinates 8j ..) and x2
// (32 + 8j ..) with the bf16 table values cw / sw (packed pairs).
__device__ __forceinline__ void rotate8(const u32x4& x1, const u32x4& x2, const uint32_t (&cw)[4],
                                        const uint32_t (&sw)[4], u32x4& y1, u32x4& y2) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float a1l = lo_f(x1[w]), a1h = hi_f(x1[w]), a2l = lo_f(x2[w]), a2h = hi_f(x2[w]);
    const float cl = lo_f(cw[w]), ch = hi_f(cw[w]), sl = lo_f(sw[w]), sh = hi_f(sw[w]);
    // each product rounded to bf16, as a separate bf16 tensor op
    const uint32_t p1c = pack_bf16(a1l * cl, a1h * ch), p2s = pack_bf16(a2l * sl, a2h * sh);
    const uint32_t p1s = pack_bf16(a1l * sl, a1h * sh), p2c = pack_bf16(a2l * cl, a2h * ch);
    y1[w] = canon_nan(pack_bf16(lo_f(p1c) - lo_f(p2s), hi_f(p1c) - hi_f(p2s)));
    y2[w] = canon_nan(pack_bf16(lo_f(p1s) + lo_f(p2c), hi_f(p1s) + hi_f(p2c)));
  }
}

// Work item: (token, head h, j) with j in 0..3: the 8 coordinate pairs
// (8j + i, 32 + 8j + i) of q and k (RoPE pairs coordinate k with k + 32) and
// the same two 16-byte pieces of v: six 16-byte loads and stores and one
// 8-pair slice of the sin / cos rows, shared by q and k. Four consecutive
// items cover a head's rows.
__global__ __launch_bounds__(256) void qkv_rope_kernel(QkvRopeArgs a) {
  const uint32_t e = wg_x() * 256u + wi_x();
  if (e >= (uint32_t)a.total) return;
  const uint32_t per_tok = 4u * (uint32_t)a.heads;
  const uint32_t tok = e / per_tok;
  const uint32_t r = e - tok * per_tok;
  const int h = (int)(r >> 2);
  const int j = (int)(r & 3u);
  const int b = (int)(tok / (uint32_t)a.seq);
  const int s = (int)tok - b * a.seq;

  const uint16_t* src = a.qkv + b * a.sx_b + s * a.sx_s + h * kHeadDim + 8 * j;
  const int64_t comp = (int64_t)a.heads * kHeadDim;  // q -> k -> v column offset
  const u32x4 q1 = ld16(src), q2 = ld16(src + kHeadDim / 2);
  const u32x4 k1 = ld16(src + comp), k2 = ld16(src + comp + kHeadDim / 2);
  const u32x4 v1 = ld16(src + 2 * comp), v2 = ld16(src + 2 * comp + kHeadDim / 2);
  int64_t pos = a.positions ? a.positions[s] : (int64_t)a.pos0 + s;
  pos = pos < 0 ? 0 : (pos >= a.max_pos ? a.max_pos - 1 : pos);  // documented clamp
  const float* cp = a.cos_t + pos * (kHeadDim / 2) + 8 * j;
  const float* sp = a.sin_t + pos * (kHeadDim / 2) + 8 * j;
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cp), c1 = *reinterpret_cast<const f32x4*>(cp + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp), s1 = *reinterpret_cast<const f32x4*>(sp + 4);

  uint16_t* vd = a.v + b * a.sv.b + h * a.sv.h + s * a.sv.s + 8 * j;
  *reinterpret_cast<u32x4*>(vd) = v1;
  *reinterpret_cast<u32x4*>(vd + kHeadDim / 2) = v2;
  // the table rows rounded to bf16 (.to(x.dtype)), two per conversion
  const uint32_t cw[4] = {pack_bf16(c0[0], c0[1]), pack_bf16(c0[2], c0[3]), pack_bf16(c1[0], c1[1]),
                          pack_bf16(c1[2], c1[3])};
  const uint32_t sw[4] = {pack_bf16(s0[0], s0[1]), pack_bf16(s0[2], s0[3]), pack_bf16(s1[0], s1[1]),
                          pack_bf16(s1[2], s1[3])};
  u32x4 y1, y2;
  rotate8(q1, q2, cw, sw, y1, y2);
  uint16_t* qd = a.q + b * a.sq.b + h * a.sq.h + s * a.sq.s + 8 * j;
  *reinterpret_cast<u32x4*>(qd) = y1;
  *reinterpret_cast<u32x4*>(qd + kHeadDim / 2) = y2;
  rotate8(k1, k2, cw, sw, y1, y2);
  uint16_t* kd = a.k + b * a.sk.b + h * a.sk.h + s * a.sk.s + 8 * j;
  *reinterpret_cast<u32x4*>(kd) = y1;
  *reinterpret_cast<u32x4*>(kd + kHeadDim / 2) = y2;
}

// One thread per 16 bytes of a head row: 8 threads per (tensor, b, h, s).
__global__ __launch_bounds__(256) void kv_write_kernel(KvWriteArgs a) {
  const int64_t e = (int64_t)wg_x() * 256 + wi_x();
  if (e >= a.total) return;
  const int part = (int)(e & 7);
  int64_t row = e >> 3;  // over (tensor, b, h, s)
  const int64_t rows = (int64_t)a.batch * a.heads * a.seq;
  const int t = row >= rows ? 1 : 0;
  row -= t * rows;
  const int s = (int)(row % a.seq);
  const int64_t bh = row / a.seq;
  const int h = (int)(bh % a.heads), b = (int)(bh / a.heads);
  const uint16_t* src = t ? a.v : a.k;
  const Strides3 ss = t ? a.sv : a.sk;
  uint16_t* dst = t ? a.v_dst : a.k_dst;
  const Strides3 sd = t ? a.svd : a.skd;
  *reinterpret_cast<u32x4*>(dst + b * sd.b + h * sd.h + s * sd.s + 8 * part) =
      ld16(src + b * ss.b + h * ss.h + s * ss.s + 8 * part);
}

}  // namespace

hipError_t launch_qkv_rope(const QkvRopeArgs& a, hipStream_t stream) {
  if (a.total == 0) return hipSuccess;
  const int64_t blocks = (a.total + 255) / 256;
  hipLaunchKernelGGL(qkv_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t stream) {
  if (a.total == 0) return hipSuccess;
  const int64_t blocks = (a.total + 255) / 256;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
