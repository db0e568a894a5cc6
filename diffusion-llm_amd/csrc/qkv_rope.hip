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
//   Work item: one (token, component, head, j) with j in 0..3 covers
//   coordinates 8j .. 8j+7 and their rotate-half partners 32+8j .. 32+8j+7
//   (RoPE pairs coordinate k with k + 32), i.e. two 16-byte loads and two
//   16-byte stores; four consecutive items cover a 128-byte head row.
//
// kv_write_kernel: the strided copy of KVCache.append (model/kv_cache.py:42-55)
//   into a preallocated cache slot instead of a torch.cat reallocation.
#include "bd3_device.h"
#include "bd3_launch.h"

namespace bd3 {
namespace {

// fp32 -> bf16 bits, round to nearest even (the conversion torch applies for
// .to(torch.bfloat16) and after every bf16 elementwise op). NaN stays NaN.
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_val(uint32_t bits) {
  return __builtin_bit_cast(float, bits << 16);
}

// The rounded value as fp32.
__device__ __forceinline__ float rnd(float f) { return bf16_val(bf16_rne(f)); }

__global__ __launch_bounds__(256) void qkv_rope_kernel(QkvRopeArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= a.total) return;
  const int per_tok = 12 * a.heads;
  const int64_t tok = e / per_tok;
  const int r = (int)(e - tok * per_tok);
  const int t = r / (4 * a.heads);  // 0 q, 1 k, 2 v
  const int h = (r >> 2) - t * a.heads;
  const int j = r & 3;
  const int b = (int)(tok / a.seq);
  const int s = (int)(tok - (int64_t)b * a.seq);

  const uint16_t* src = a.qkv + b * a.sx_b + s * a.sx_s + (t * a.heads + h) * kHeadDim + 8 * j;
  const u32x4 x1 = ld16(src);
  const u32x4 x2 = ld16(src + kHeadDim / 2);
  uint16_t* out = t == 0 ? a.q : (t == 1 ? a.k : a.v);
  const Strides3 so = t == 0 ? a.sq : (t == 1 ? a.sk : a.sv);
  uint16_t* dst = out + b * so.b + h * so.h + s * so.s + 8 * j;
  if (t == 2) {
    *reinterpret_cast<u32x4*>(dst) = x1;
    *reinterpret_cast<u32x4*>(dst + kHeadDim / 2) = x2;
    return;
  }
  int64_t pos = a.positions ? a.positions[s] : (int64_t)a.pos0 + s;
  pos = pos < 0 ? 0 : (pos >= a.max_pos ? a.max_pos - 1 : pos);  // documented clamp
  const float* cp = a.cos_t + pos * (kHeadDim / 2) + 8 * j;
  const float* sp = a.sin_t + pos * (kHeadDim / 2) + 8 * j;
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cp), c1 = *reinterpret_cast<const f32x4*>(cp + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp), s1 = *reinterpret_cast<const f32x4*>(sp + 4);
  const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  u32x4 y1, y2;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t lo1 = 0, lo2 = 0;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int i = 2 * w + half;
      const float a1 = bf16_val((x1[w] >> (16 * half)) & 0xffffu);
      const float a2 = bf16_val((x2[w] >> (16 * half)) & 0xffffu);
      const float c = rnd(cs[i]), sv = rnd(sn[i]);
      const uint32_t o1 = bf16_rne(rnd(a1 * c) - rnd(a2 * sv));
      const uint32_t o2 = bf16_rne(rnd(a1 * sv) + rnd(a2 * c));
      lo1 |= o1 << (16 * half);
      lo2 |= o2 << (16 * half);
    }
    y1[w] = lo1;
    y2[w] = lo2;
  }
  *reinterpret_cast<u32x4*>(dst) = y1;
  *reinterpret_cast<u32x4*>(dst + kHeadDim / 2) = y2;
}

// One thread per 16 bytes of a head row: 8 threads per (tensor, b, h, s).
__global__ __launch_bounds__(256) void kv_write_kernel(KvWriteArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
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
