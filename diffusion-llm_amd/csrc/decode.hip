// decode.hip - BD3-LM decode attention over the KV cache for gfx950.
//
// Counterpart of block_sparse_decode_kern (kernels/BlockSparseDecodeAttention.py:40-110)
// and split_kv_kern / split_kv_reduce_kern (kernels/SplitKVDecodeAttention.py:16-127).
// Queries are the last q_len of kv_len positions; row i sees key j iff
// j / bs <= (kv_len - q_len + i) / bs and j < kv_len (bd3_mask.h).
//
// decode_partial: one workgroup per (split, 32-row query tile, batch*head).
//   The split's key range is cut into 64-key chunks that the four waves take
//   in turn; each wave runs an online softmax over its chunks, then the four
//   states are merged through LDS. With one split the workgroup writes O
//   directly; otherwise it writes a normalised fp32 partial and its log2-LSE.
//   S^T (32 keys x 32 rows) = K Q^T on v_mfma_f32_32x32x16_bf16 with K read
//   from HBM straight into A-operand registers (one 16-byte load per lane and
//   operand: a 128-byte key row is covered by 8 consecutive lanes' loads);
//   V goes through a wave-private row-major LDS tile and is read transposed
//   (ds_read_b64_tr_b16) as the A operand of O^T += V^T P^T.
// decode_combine: merges the splits, weights exp2(lse_s - max lse) (the
//   reference's split_kv_reduce_kern arithmetic, :109-127).
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"

namespace bd3 {
namespace {

constexpr int kNW = 4;
constexpr int kThreads = kNW * 64;
constexpr int kQT = 32;       // query rows per workgroup
constexpr int kChunk = 64;    // keys per wave step
constexpr int kStride = 72;   // padded LDS row (bf16)
constexpr int kVElems = kChunk * kStride;

struct MergeLds {
  float o[kNW][kHeadDim][kQT + 1];  // O^T per wave (unnormalised), padded
  float m[kNW][kQT];
  float l[kNW][kQT];
};
constexpr size_t kVBytes = sizeof(__bf16) * kNW * kVElems;
constexpr size_t kSmemBytes = kVBytes > sizeof(MergeLds) ? kVBytes : sizeof(MergeLds);

__global__ __launch_bounds__(kThreads) void decode_partial(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  __bf16* vs = reinterpret_cast<__bf16*>(smem) + (threadIdx.x >> 6) * kVElems;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int split = blockIdx.x;
  const int qt = blockIdx.y;
  const int bh = blockIdx.z;
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int i0 = qt * kQT;

  const uint16_t* qp = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* kp = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vp = a.v + b * a.sv.b + h * a.sv.h;

  // Q^T B operand: lane holds row i0 + l32 (clamped), d = 16c + 8g .. +7.
  const int myi = i0 + l32;
  const int qrow = imin(myi, a.q_len - 1);
  bf16x8 qreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qreg[c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)qrow * a.sq.s + 16 * c + 8 * g));
  // Row i sees keys [0, khi).
  const int pos = a.kv_len - a.q_len + myi;
  const int khi = imin((pos / a.bs + 1) * a.bs, a.kv_len);

  const int key_end = decode_key_end(i0, kQT, a.q_len, a.kv_len, a.bs);
  const int lo = split * a.split_len;
  const int hi = imin(lo + a.split_len, key_end);
  const int n_chunks = hi > lo ? (hi - lo + kChunk - 1) / kChunk : 0;

  f32x16 oacc[2] = {};
  float m = -INFINITY, lsum = 0.f;

  for (int ch = wave; ch < n_chunks; ch += kNW) {
    const int c0 = lo + ch * kChunk;
    // K A-operands for the two 32-key sub-blocks (rows clamped in-bounds).
    bf16x8 kop[2][4];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int key = imin(c0 + 32 * sb + l32, a.kv_len - 1);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kop[sb][c] = __builtin_bit_cast(bf16x8, ld16(kp + (int64_t)key * a.sk.s + 16 * c + 8 * g));
    }
    // V chunk -> wave-private LDS (row-major), 8 lanes per 128-byte row.
    u32x4 vbuf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane + 64 * j;
      const int key = imin(c0 + (e >> 3), a.kv_len - 1);
      vbuf[j] = ld16(vp + (int64_t)key * a.sv.s + (e & 7) * 8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane + 64 * j;
      *reinterpret_cast<u32x4*>(&vs[(e >> 3) * kStride + (e & 7) * 8]) = vbuf[j];
    }

    int cls[2];
    f32x16 s[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int j0 = c0 + 32 * sb;
      // keys past hi belong to the next split (or are invisible)
      cls[sb] = j0 >= hi ? kNone : decode_class(i0, kQT, j0, 32, a.q_len, a.kv_len, a.bs);
      if (cls[sb] == kFull && j0 + 32 > hi) cls[sb] = kPartial;
      s[sb] = f32x16{};
      if (cls[sb] != kNone) {
#pragma unroll
        for (int c = 0; c < 4; ++c) s[sb] = mfma32(kop[sb][c], qreg[c], s[sb]);
        if (cls[sb] == kPartial) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = j0 + 8 * (r >> 2) + 4 * g + (r & 3);
            if (key >= khi || key >= hi) s[sb][r] = -INFINITY;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[sb][r] = -INFINITY;
      }
    }
    if (cls[0] == kNone && cls[1] == kNone) continue;

    float mx = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
    mx = max_xor32(mx);
    const float m_new = fmaxf(m, mx * a.scale_log2);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    m = m_new;
    lsum *= alpha;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;

    const int tr_row = (lane & 15) >> 2;
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (cls[sb] == kNone) continue;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = fast_exp2(fmaf(s[sb][r], a.scale_log2, -m_use));
        lsum += p[r];
      }
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const bf16x8 pop = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3],
                                     p[8 * kc + 4], p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
        const int row = 32 * sb + 16 * kc + 4 * g + tr_row;
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 va = cat8(lds_read_tr(&vs[row * kStride + 32 * db + tr_col]),
                                 lds_read_tr(&vs[(row + 8) * kStride + 32 * db + tr_col]));
          oacc[db] = mfma32(va, pop, oacc[db]);
        }
      }
    }
  }

  // Merge the four waves' states.
  lsum = sum_xor32(lsum);
  __syncthreads();  // V staging area is reused below
  MergeLds* ml = reinterpret_cast<MergeLds*>(smem);
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
      ml->o[wave][d][l32] = oacc[db][r];
    }
  if (g == 0) {
    ml->m[wave][l32] = m;
    ml->l[wave][l32] = lsum;
  }
  __syncthreads();

  const int split_out = a.n_splits > 1;
  uint16_t* op = a.o + b * a.so.b + h * a.so.h;
  const int64_t slot = ((int64_t)bh * a.q_tiles + qt) * a.n_splits + split;
#pragma unroll
  for (int j = 0; j < (kQT * kHeadDim) / kThreads; ++j) {
    const int e = tid + kThreads * j;
    const int row = e >> 6, d = e & 63;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kNW; ++w) mm = fmaxf(mm, ml->m[w][row]);
    const float mu = (mm == -INFINITY) ? 0.f : mm;
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int w = 0; w < kNW; ++w) {
      const float wgt = fast_exp2(ml->m[w][row] - mu);
      lt += wgt * ml->l[w][row];
      ot += wgt * ml->o[w][d][row];
    }
    if (!split_out) {
      if (i0 + row < a.q_len) {
        const __bf16 y = (__bf16)(ot / lt);
        op[(int64_t)(i0 + row) * a.so.s + d] = __builtin_bit_cast(uint16_t, y);
      }
    } else {
      a.part_o[(slot * kQT + row) * kHeadDim + d] = lt > 0.f ? ot / lt : 0.f;
      if (d == 0) a.part_lse[slot * kQT + row] = lt > 0.f ? mm + fast_log2(lt) : -INFINITY;
    }
  }
}

__global__ __launch_bounds__(kThreads) void decode_combine(DecodeArgs a) {
  const int qt = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int i0 = qt * kQT;
  uint16_t* op = a.o + b * a.so.b + h * a.so.h;
  const int64_t slot0 = ((int64_t)bh * a.q_tiles + qt) * a.n_splits;
#pragma unroll
  for (int j = 0; j < (kQT * kHeadDim) / kThreads; ++j) {
    const int e = threadIdx.x + kThreads * j;
    const int row = e >> 6, d = e & 63;
    if (i0 + row >= a.q_len) continue;
    float mm = -INFINITY;
    for (int s = 0; s < a.n_splits; ++s) mm = fmaxf(mm, a.part_lse[(slot0 + s) * kQT + row]);
    float wt = 0.f, acc = 0.f;
    for (int s = 0; s < a.n_splits; ++s) {
      const float lse = a.part_lse[(slot0 + s) * kQT + row];
      const float w = fast_exp2(lse - mm);  // -inf lse (empty split) -> 0
      wt += w;
      acc += w * a.part_o[((slot0 + s) * kQT + row) * kHeadDim + d];
    }
    const __bf16 y = (__bf16)(acc / wt);
    op[(int64_t)(i0 + row) * a.so.s + d] = __builtin_bit_cast(uint16_t, y);
  }
}

__global__ void mask_dump_kernel(uint8_t* out, int mode, int rows, int cols, int kv_len,
                                 int bs) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)rows * cols) return;
  const int i = (int)(e / cols), j = (int)(e - (int64_t)i * cols);
  bool vis;
  if (mode == 0) {
    vis = train_visible(i, j, rows / 2, bs);
  } else {
    vis = decode_visible(i, j, rows, kv_len, bs);
  }
  out[e] = vis ? 1 : 0;
}

}  // namespace

hipError_t launch_decode(const DecodeArgs& a, int /*qt*/, hipStream_t stream) {
  dim3 grid(a.n_splits, a.q_tiles, a.bh);
  hipLaunchKernelGGL(decode_partial, grid, dim3(kThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.n_splits == 1) return e;
  hipLaunchKernelGGL(decode_combine, dim3(a.q_tiles, a.bh), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_mask_dump(uint8_t* out, int mode, int rows, int kv_len, int bs,
                            hipStream_t stream) {
  const int r = mode == 0 ? 2 * rows : rows;
  const int c = mode == 0 ? 2 * rows : kv_len;
  const int64_t total = (int64_t)r * c;
  hipLaunchKernelGGL(mask_dump_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                     out, mode, r, c, kv_len, bs);
  return hipGetLastError();
}

}  // namespace bd3
