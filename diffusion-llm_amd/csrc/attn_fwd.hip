// attn_fwd.hip - BD3-LM training attention forward for gfx950.
//
// O = softmax(Q K^T * scale + M) V over cat(x_t, x_0) (length 2n), M the
// block-diffusion mask (bd3_mask.h). Counterpart of
// block_sparse_attention_fwd_kern (kernels/BlockSparseFlashAttention.py:75-172).
//
// Work split: one workgroup per (batch*head, 128-row query tile), four
// waves of 32 rows each. A query tile lies entirely in one half (n % 128 == 0).
// Key tiles of 64 keys are staged through LDS (double-buffered, row-major,
// padded) and visited only where the mask has live pairs for the workgroup
// (train_key_ranges); each wave further skips 32-key sub-blocks that are dead
// for its own rows and masks only partial ones (train_class).
//
// Per wave and 32-key sub-block:
//   S^T (32 keys x 32 rows) = K Q^T on v_mfma_f32_32x32x16_bf16. A lane then
//   holds one query row (lane % 32) and 16 of its keys, so the online-softmax
//   statistics are lane-local up to one permlane32 exchange.
//   O^T (64 x 32) += V^T P^T, with V^T read from the row-major LDS tile by
//   ds_read_b64_tr_b16 and P^T taken straight from the S^T registers (the key
//   order inside the MFMA reduction is permuted identically on both sides).
// The softmax runs in base 2 with scale*log2(e) folded into one FMA; lse is
// written in natural log as the reference does (L = m + log l, :166-172).
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"

namespace bd3 {
namespace {

constexpr int kNW = 4;            // waves per workgroup
constexpr int kBM = 32 * kNW;     // query rows per workgroup
constexpr int kBN = 64;           // keys per LDS tile
constexpr int kLdsStride = 72;    // bf16 per LDS row (64 + 8 pad: conflict-free b128 reads)
constexpr int kTileElems = kBN * kLdsStride;
constexpr int kThreads = kNW * 64;
constexpr int kChunks = (kBN * kHeadDim / 8) / kThreads;  // 16-B chunks per thread per tensor

__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][kTileElems];  // [stage][K|V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;  // lane half

  // Heaviest query tiles first (the last tiles of each half see the most
  // keys); within a rank, consecutive workgroups walk batch*head so that all
  // tiles of one (b, h) land on the same XCD when bh % 8 == 0.
  const int tiles_half = a.n / kBM;
  const int rank = blockIdx.x / a.bh;
  const int bh = blockIdx.x - rank * a.bh;
  const int t = tiles_half - 1 - (rank >> 1);
  const int half = (rank & 1) ? 0 : 1;  // clean tiles first at equal rank
  const int q0 = half * a.n + t * kBM;
  const int b = bh / a.heads, h = bh - b * a.heads;

  const uint16_t* qp = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* kp = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vp = a.v + b * a.sv.b + h * a.sv.h;

  // Q^T as the B operand: lane holds row (qrow0 + l32), d = 16c + 8g .. +7.
  const int qrow0 = q0 + wave * 32;
  const int myq = qrow0 + l32;
  const RowIntervals riv = train_row_intervals(myq, a.n, a.bs);
  bf16x8 qreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4 raw = ld16(qp + (int64_t)myq * a.sq.s + 16 * c + 8 * g);
    qreg[c] = __builtin_bit_cast(bf16x8, raw);
  }

  const KeyRanges kr = train_key_ranges(q0, kBM, a.n, a.bs, kBN);
  const int n_first = kr.t1 - kr.t0;
  const int n_tiles = n_first + (kr.t3 - kr.t2);

  // Cooperative tile load: chunk c -> key c/8, 16-B part c%8 (coalesced rows).
  u32x4 kbuf[kChunks], vbuf[kChunks];
  auto tile_of = [&](int i) { return i < n_first ? kr.t0 + i : kr.t2 + (i - n_first); };
  auto load_tile = [&](int i) {
    const int k0 = tile_of(i) * kBN;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * kThreads;
      const int key = k0 + (c >> 3);
      const int col = (c & 7) * 8;
      kbuf[j] = ld16(kp + (int64_t)key * a.sk.s + col);
      vbuf[j] = ld16(vp + (int64_t)key * a.sv.s + col);
    }
  };
  auto store_tile = [&](int stage) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * kThreads;
      const int off = (c >> 3) * kLdsStride + (c & 7) * 8;
      *reinterpret_cast<u32x4*>(&smem[stage][0][off]) = kbuf[j];
      *reinterpret_cast<u32x4*>(&smem[stage][1][off]) = vbuf[j];
    }
  };

  f32x16 oacc[2] = {};  // O^T blocks: d rows [32*db, 32*db+32), query column l32
  float m = -INFINITY;  // running max of scaled scores (log2 domain)
  float lsum = 0.f;     // lane-local partial row sum

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int stage = it & 1;
    if (it + 1 < n_tiles) load_tile(it + 1);

    const int k0 = tile_of(it) * kBN;
    const __bf16* ks = smem[stage][0];
    const __bf16* vs = smem[stage][1];

    int cls[2];
    cls[0] = train_class(qrow0, 32, k0, 32, a.n, a.bs);
    cls[1] = train_class(qrow0, 32, k0 + 32, 32, a.n, a.bs);

    if (cls[0] != kNone || cls[1] != kNone) {
      f32x16 s[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        s[sb] = f32x16{};
        if (cls[sb] != kNone) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const bf16x8 kop = *reinterpret_cast<const bf16x8*>(
                &ks[(32 * sb + l32) * kLdsStride + 16 * c + 8 * g]);
            s[sb] = mfma32(kop, qreg[c], s[sb]);
          }
          if (cls[sb] == kPartial) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = k0 + 32 * sb + 8 * (r >> 2) + 4 * g + (r & 3);
              if (!row_sees(riv, key)) s[sb][r] = -INFINITY;
            }
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) s[sb][r] = -INFINITY;
        }
      }

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
          const bf16x8 pop = to_bf16x8(p[8 * kc + 0], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3],
                                       p[8 * kc + 4], p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
          // V^T operand: lane group G = lane/16 reads key rows
          // 32sb + 16kc + 4g + (lane%16)/4 (and +8), columns 32db + 16(G%2) + 4(lane%4).
          const int row = 32 * sb + 16 * kc + 4 * g + ((lane & 15) >> 2);
          const int colb = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
          for (int db = 0; db < 2; ++db) {
            const bf16x4 lo = lds_read_tr(&vs[row * kLdsStride + 32 * db + colb]);
            const bf16x4 hi = lds_read_tr(&vs[(row + 8) * kLdsStride + 32 * db + colb]);
            oacc[db] = mfma32(cat8(lo, hi), pop, oacc[db]);
          }
        }
      }
    }

    if (it + 1 < n_tiles) store_tile(stage ^ 1);
    __syncthreads();
  }

  // Epilogue: O = O^T / l, lse = (m + log2 l) * ln 2.
  const float ltot = sum_xor32(lsum);
  const float inv = 1.f / ltot;
  uint16_t* op = a.o + b * a.so.b + h * a.so.h + (int64_t)myq * a.so.s;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int d = 32 * db + 8 * rg + 4 * g;
      const bf16x4 v4 = to_bf16x4(oacc[db][4 * rg] * inv, oacc[db][4 * rg + 1] * inv,
                                  oacc[db][4 * rg + 2] * inv, oacc[db][4 * rg + 3] * inv);
      *reinterpret_cast<bf16x4*>(op + d) = v4;
    }
  if (g == 0) a.lse[(int64_t)bh * 2 * a.n + myq] = (m + fast_log2(ltot)) * kLn2;
}

}  // namespace

hipError_t launch_attn_fwd(const FwdArgs& a, hipStream_t stream) {
  const int grid = a.bh * (2 * a.n / kBM);
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(grid), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
